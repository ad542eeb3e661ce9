"""Several GPU jobs in flight at once, each on a stream of its own.

Some host paths size their next launch from a count the GPU has just
computed (a product total, an output length), so each such step waits for a
device-to-host copy.  One job at a time, the GPU idles through every one of
those round trips.  Here a job is a generator function ``job(stream, host)``
that enqueues its work on ``stream``, copies the count it needs into
``host`` (pinned int64 host memory) asynchronously, records an event and
yields; resumed, it waits for that event and goes on.  Its return value
(a tensor or a tuple of them) is its result.  ``run_in_flight`` keeps up to
``streams`` jobs going round robin, so one job's wait overlaps the other
jobs' kernels.  The streams keep the default priority.
"""
from __future__ import annotations

import collections

import torch

_STREAMS: dict = {}


def side_streams(device: torch.device, n: int) -> list:
    """n streams of default priority on ``device``, created once per process
    and reused by every call."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    have = _STREAMS.setdefault(idx, [])
    while len(have) < n:
        have.append(torch.cuda.Stream(torch.device("cuda", idx)))
    return have[:n]


def run_in_flight(jobs, device, streams: int, host_len: int = 2) -> list:
    """Runs ``jobs`` (see the module docstring) with up to ``streams`` in
    flight; 1 runs them one after another on the current stream.  Returns
    their results in job order, ready on the current stream.  Work that a
    job's inputs need must be enqueued on the current stream before the
    call.  On an error the current stream still waits for everything the
    jobs enqueued, so later work cannot overwrite memory they still use."""
    if not jobs:
        return []
    dev = torch.device(device)
    cur = torch.cuda.current_stream(dev)
    n_str = max(1, min(int(streams), len(jobs)))
    pool = [cur] if n_str == 1 else side_streams(dev, n_str)
    hosts = [torch.empty(host_len, dtype=torch.int64, pin_memory=True) for _ in pool]
    results = [None] * len(jobs)
    queue = iter(enumerate(jobs))

    def start(slot):
        nxt = next(queue, None)
        if nxt is None:
            return None
        i, job = nxt
        pool[slot].wait_stream(cur)  # the job's inputs come from the current stream
        return job(pool[slot], hosts[slot]), i, slot

    try:
        active = collections.deque(e for e in map(start, range(n_str)) if e is not None)
        while active:
            entry = active.popleft()
            try:
                next(entry[0])
                active.append(entry)
            except StopIteration as stop:
                results[entry[1]] = stop.value
                nxt = start(entry[2])
                if nxt is not None:
                    active.append(nxt)
    finally:
        for s in pool:
            cur.wait_stream(s)
    if n_str > 1:
        for r in results:
            for t in (r if isinstance(r, tuple) else (r,)):
                if isinstance(t, torch.Tensor):
                    t.record_stream(cur)
    return results
