"""Read scheduling and prompt-tail retention for the slot cache: the reference's
qwen_streaming_policy.py (runtime/deepseek_v4_ssd/qwen_streaming_policy.py:7-45), same
functions and errors. They never change routes."""
from __future__ import annotations

import numpy as np


def contiguous_batches(experts, maximum: int):
    """Split sorted unique expert ids into runs of consecutive ids of at most `maximum`
    (1..32), in order: each run is one contiguous read (qwen_streaming_policy.py:7-20)."""
    if type(maximum) is not int or not 1 <= maximum <= 32:
        raise ValueError("read batch size must be an integer from 1 through 32")
    ids = tuple(experts)
    if any(type(i) is not int or i < 0 for i in ids):
        raise ValueError("expert IDs must be nonnegative integers")
    if any(b <= a for a, b in zip(ids, ids[1:])):
        raise ValueError("expert IDs must be sorted and unique")
    run = []
    for i in ids:
        if run and (len(run) == maximum or i != run[-1] + 1):
            yield tuple(run)
            run = []
        run.append(i)
    if run:
        yield tuple(run)


def hot_tail_experts(routes, expert_count: int, limit: int):
    """The experts of the last 128 routed positions, ranked by count, then by most recent
    use, then by id; up to `limit` of them returned least valuable first, so seeding them
    in order leaves the hottest most recent (qwen_streaming_policy.py:23-45)."""
    if type(limit) is not int or limit < 0 or type(expert_count) is not int or expert_count < 1:
        raise ValueError("invalid prefill retention dimensions")
    rows = np.asarray(routes)
    if rows.ndim not in (2, 3) or rows.dtype.kind not in "iu" or rows.shape[-1] < 1:
        raise ValueError("routes must be integer token-by-expert rows")
    if rows.size and (rows.min() < 0 or rows.max() >= expert_count):
        raise ValueError("routed expert outside model range")
    tail = rows.reshape(-1, rows.shape[-1])[-128:].reshape(-1).astype(np.int64)
    if tail.size == 0 or limit == 0:
        return []
    count = np.bincount(tail, minlength=expert_count)
    last = np.full(expert_count, -1, np.int64)
    np.maximum.at(last, tail, np.arange(tail.size))  # each expert's latest position
    seen = np.flatnonzero(count)
    best = seen[np.lexsort((seen, -last[seen], -count[seen]))][:limit]
    return best[::-1].tolist()
