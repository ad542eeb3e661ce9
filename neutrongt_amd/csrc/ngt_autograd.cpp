// C++ autograd node of the sparse window attention.
//
// The same operation and contract as SparseAttentionFunction in attention.py
// (the reference op is CoreAttention.sparse_attention_bias,
// NeutronGT/models/graphormer_dist_node_level.py:67-98): (q, k, v) ->
// (out, node_scores), node scores without gradient, optional detached extra
// key rows (k_ext, v_ext).  Forward and backward call the library's C ABI
// (ngt_sparse_fwd_ext / ngt_sparse_bwd_strided) through function pointers that the
// Python side hands over once from the loaded libngt_attn.so, so a layer's
// forward and backward run no Python frame, take no GIL on the autograd
// engine's device thread and convert no ctypes arguments.  Host code only:
// every kernel is in libngt_attn.so.
//
// The window is passed as two tensors: `csr` (CPU bytes of one
// ngt_window_csr) and `csr_mem` (the device allocation its pointers point
// into).  Both are kept by the node until the backward has run.
#include <torch/extension.h>

#include <c10/hip/HIPStream.h>

#include "ngt_attn.h"

namespace {

using at::Tensor;
using torch::autograd::AutogradContext;
using torch::autograd::tensor_list;

decltype(&ngt_sparse_fwd_ext) g_fwd = nullptr;
decltype(&ngt_sparse_bwd_strided) g_bwd = nullptr;
decltype(&ngt_last_error) g_err = nullptr;

void check(int rc) {
  if (rc != NGT_OK) {
    const char* msg = g_err ? g_err() : nullptr;
    TORCH_CHECK(!(msg && *msg), msg);
    TORCH_CHECK(false, "libngt_attn error ", rc);
  }
}

int dtype_code(const Tensor& t) {
  if (t.scalar_type() == at::kFloat) return NGT_F32;
  if (t.scalar_type() == at::kBFloat16) return NGT_BF16;
  TORCH_CHECK(false, "unsupported dtype ", t.scalar_type(), " (float32 or bfloat16)");
  return -1;
}

void* stream_of(const Tensor& t) {
  return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

const ngt_window_csr* csr_of(const Tensor& bytes) {
  return reinterpret_cast<const ngt_window_csr*>(bytes.data_ptr());
}

// 16-byte aligned contiguous rows, as the library requires
Tensor rows16(const Tensor& t) {
  if (!t.is_contiguous()) return t.contiguous();
  if (reinterpret_cast<uintptr_t>(t.data_ptr()) % 16) return t.clone();
  return t;
}

// The library reads rows [n, H, d] of one dtype from 16-byte aligned,
// contiguous GPU memory on q's device; anything else is an error here rather
// than wrong reads in the kernels.
void check_rows(const char* name, const Tensor& t, const Tensor& q) {
  TORCH_CHECK(t.is_cuda(), name, " must be a GPU tensor");
  TORCH_CHECK(t.device() == q.device(), name, " is on ", t.device(), ", q on ", q.device());
  TORCH_CHECK(t.scalar_type() == q.scalar_type(), name, " has dtype ", t.scalar_type(),
              ", q has ", q.scalar_type());
  TORCH_CHECK(t.dim() == 3 && t.size(1) == q.size(1) && t.size(2) == q.size(2), name,
              " must be [n, ", q.size(1), ", ", q.size(2), "], got ", t.sizes());
  TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
  TORCH_CHECK(reinterpret_cast<uintptr_t>(t.data_ptr()) % 16 == 0, name,
              " must be 16-byte aligned");
}

Tensor workspace(int64_t bytes, const Tensor& like) {
  return at::empty({std::max<int64_t>(bytes, 1)}, like.options().dtype(at::kByte));
}

constexpr int kInputs = 15;  // forward arguments after ctx

struct SparseAttention : public torch::autograd::Function<SparseAttention> {
  static tensor_list forward(AutogradContext* ctx, Tensor q, Tensor k, Tensor v,
                             std::optional<Tensor> k_ext_opt, std::optional<Tensor> v_ext_opt,
                             Tensor csr, Tensor csr_mem, int64_t dst_end,
                             double scale, double lo, double hi, double eps, int64_t fwd_bytes,
                             int64_t bwd_bytes, bool interleave_grads) {
    TORCH_CHECK(g_fwd && g_bwd, "ngt_autograd.init() was not called");
    // an absent argument is an empty optional: autograd inputs may not be
    // undefined tensors
    const Tensor k_ext = k_ext_opt.value_or(Tensor()), v_ext = v_ext_opt.value_or(Tensor());
    const bool ext = k_ext.defined();
    TORCH_CHECK(ext == v_ext.defined(), "k_ext and v_ext must be given together");
    check_rows("q", q, q);
    check_rows("k", k, q);
    check_rows("v", v, q);
    TORCH_CHECK(k.sizes() == v.sizes(), "k and v differ in shape: ", k.sizes(), " vs ", v.sizes());
    if (ext) {
      check_rows("k_ext", k_ext, q);
      check_rows("v_ext", v_ext, q);
      TORCH_CHECK(k_ext.sizes() == v_ext.sizes(), "k_ext and v_ext differ in shape");
    }
    const int64_t n_q = q.size(0), H = q.size(1), d = q.size(2);
    Tensor out = at::empty_like(q);
    const auto f32 = q.options().dtype(at::kFloat);
    Tensor rinv = at::empty({n_q, H}, f32);
    Tensor ns = at::empty({dst_end}, f32);
    Tensor ws = workspace(fwd_bytes, q);
    check(g_fwd(dtype_code(q), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                ext ? k_ext.data_ptr() : nullptr, ext ? v_ext.data_ptr() : nullptr,
                static_cast<int32_t>(k.size(0)), csr_of(csr), static_cast<int32_t>(H),
                static_cast<int32_t>(d), static_cast<float>(scale), static_cast<float>(lo),
                static_cast<float>(hi), static_cast<float>(eps), out.data_ptr(),
                rinv.data_ptr<float>(), dst_end ? ns.data_ptr<float>() : nullptr,
                static_cast<int32_t>(dst_end), ws.data_ptr(), static_cast<size_t>(fwd_bytes),
                stream_of(q)));
    ctx->save_for_backward({q, k, v, out, rinv});
    ctx->saved_data["k_ext"] = k_ext;  // detached key rows (no gradient)
    ctx->saved_data["v_ext"] = v_ext;
    ctx->saved_data["csr"] = csr;
    ctx->saved_data["csr_mem"] = csr_mem;
    ctx->saved_data["scale"] = scale;
    ctx->saved_data["lo"] = lo;
    ctx->saved_data["hi"] = hi;
    ctx->saved_data["bwd_bytes"] = bwd_bytes;
    ctx->saved_data["interleave"] = interleave_grads && n_q == k.size(0);
    ctx->mark_non_differentiable({ns});
    // the node scores have no gradient: no zero tensor is made for them
    ctx->set_materialize_grads(false);
    return {out, ns};
  }

  static tensor_list backward(AutogradContext* ctx, tensor_list grads) {
    tensor_list res(kInputs);
    if (!grads[0].defined()) return res;  // the output was not used by the loss
    const auto saved = ctx->get_saved_variables();
    const Tensor &q = saved[0], &k = saved[1], &v = saved[2], &out = saved[3], &rinv = saved[4];
    const Tensor k_ext = ctx->saved_data["k_ext"].toTensor();
    const Tensor v_ext = ctx->saved_data["v_ext"].toTensor();
    const Tensor csr = ctx->saved_data["csr"].toTensor();
    const int64_t bwd_bytes = ctx->saved_data["bwd_bytes"].toInt();
    const Tensor g = rows16(grads[0].to(q.scalar_type()));
    Tensor gq, gk, gv;
    int64_t ldg = 0;
    if (ctx->saved_data["interleave"].toBool()) {
      // one [N, 3, H, d] buffer: row i holds dQ, dK, dV of row i side by side
      const Tensor buf = at::empty({q.size(0), 3, q.size(1), q.size(2)}, q.options());
      gq = buf.select(1, 0);
      gk = buf.select(1, 1);
      gv = buf.select(1, 2);
      ldg = 3 * q.size(1) * q.size(2);
    } else {
      gq = at::empty_like(q);
      gk = at::empty_like(k);
      gv = at::empty_like(v);
    }
    Tensor ws = workspace(bwd_bytes, q);
    const bool ext = k_ext.defined();
    check(g_bwd(dtype_code(q), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                ext ? k_ext.data_ptr() : nullptr, ext ? v_ext.data_ptr() : nullptr,
                static_cast<int32_t>(k.size(0)), out.data_ptr(), g.data_ptr(),
                rinv.data_ptr<float>(), csr_of(csr), static_cast<int32_t>(q.size(1)),
                static_cast<int32_t>(q.size(2)),
                static_cast<float>(ctx->saved_data["scale"].toDouble()),
                static_cast<float>(ctx->saved_data["lo"].toDouble()),
                static_cast<float>(ctx->saved_data["hi"].toDouble()), gq.data_ptr(),
                gk.data_ptr(), gv.data_ptr(), ldg, ws.data_ptr(), static_cast<size_t>(bwd_bytes),
                stream_of(q)));
    res[0] = gq;
    res[1] = gk;
    res[2] = gv;
    return res;
  }
};

std::tuple<Tensor, Tensor> sparse_attention(Tensor q, Tensor k, Tensor v,
                                            std::optional<Tensor> k_ext,
                                            std::optional<Tensor> v_ext, Tensor csr,
                                            Tensor csr_mem, int64_t dst_end, double scale,
                                            double lo, double hi, double eps, int64_t fwd_bytes,
                                            int64_t bwd_bytes, bool interleave_grads) {
  TORCH_CHECK(csr.device().is_cpu() && csr.scalar_type() == at::kByte &&
                  csr.numel() == static_cast<int64_t>(sizeof(ngt_window_csr)),
              "csr must hold the bytes of one ngt_window_csr (", sizeof(ngt_window_csr), ")");
  auto r = SparseAttention::apply(q, k, v, k_ext, v_ext, csr, csr_mem, dst_end, scale, lo, hi, eps,
                                  fwd_bytes, bwd_bytes, interleave_grads);
  return {r[0], r[1]};
}

void init(int64_t fwd, int64_t bwd, int64_t err) {
  g_fwd = reinterpret_cast<decltype(&ngt_sparse_fwd_ext)>(fwd);
  g_bwd = reinterpret_cast<decltype(&ngt_sparse_bwd_strided)>(bwd);
  g_err = reinterpret_cast<decltype(&ngt_last_error)>(err);
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("init", &init, "entry points of libngt_attn.so: fwd, bwd, last_error (addresses)");
  m.def("csr_struct_bytes", []() { return static_cast<int64_t>(sizeof(ngt_window_csr)); });
  m.def("abi_version", []() { return static_cast<int64_t>(NGT_ABI_VERSION); },
        "NGT_ABI_VERSION of the header this extension was compiled against");
  m.def("sparse_attention", &sparse_attention,
        "(q, k, v, k_ext, v_ext, csr, csr_mem, dst_end, scale, lo, hi, eps, fwd_bytes, "
        "bwd_bytes, interleave_grads) -> (out, node_scores); interleave_grads: dQ, dK, dV as "
        "views of one [N, 3, H, d] buffer (when q and k have the same rows)");
}
