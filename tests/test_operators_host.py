"""Host logic of the operator mirrors (whallm_amd/operators.py), CPU only: weight
containers -> expert tables, the duck-typed cache protocol, id compaction and the
reference's error behaviour. No kernel runs here (tables are built from CPU tensors)."""
from types import SimpleNamespace

import pytest
import torch

from whallm_amd import operators as O
from whallm_amd.ops import MXFP4Experts


def _qwen_expert(value: int, H=64, I=32):
    return O.QwenExpertWeights(
        torch.full((2 * I, H // 8), value, dtype=torch.int32), torch.full((2 * I, H // 32), 127, dtype=torch.uint8),
        torch.full((H, I // 8), value, dtype=torch.int32), torch.full((H, I // 32), 127, dtype=torch.uint8))


def _deepseek_expert(value: int, H=64, I=32, fused=False):
    w = lambda rows, cols, v: torch.full((rows, cols // 8), v, dtype=torch.int32)  # noqa: E731
    s = lambda rows, cols: torch.full((rows, cols // 32), 127, dtype=torch.uint8)  # noqa: E731
    e = O.ExpertWeights(w(I, H, value), s(I, H), w(H, I, value + 1), s(H, I), w(I, H, value + 2), s(I, H))
    if fused:
        e = O.ExpertWeights(e.w1, e.w1_scales, e.w2, e.w2_scales, e.w3, e.w3_scales,
                            torch.cat([e.w3, e.w1]), torch.cat([e.w3_scales, e.w1_scales]))
    return e


def test_qwen_container_is_gate_first_table():
    t = O._as_table(_qwen_expert(5))
    assert isinstance(t, MXFP4Experts) and not t.up_first
    assert (t.hidden, t.inter) == (64, 32)


@pytest.mark.parametrize("fused", [False, True])
def test_deepseek_container_is_up_first_w13(fused):
    e = _deepseek_expert(1, fused=fused)
    t = O._as_table(e, 10.0)
    assert t.up_first and t.swiglu_limit == 10.0
    # rows 0..I-1 are w3 (up), I..2I-1 are w1 (gate) (expert_layout.py:43-51)
    assert int(t.gate_up[0, 0]) == 3 and int(t.gate_up[32, 0]) == 1


def test_get_many_gathers_a_compact_table_and_records_the_sync():
    experts = {e: _qwen_expert(e) for e in range(6)}
    calls = []
    cache = SimpleNamespace(
        model=SimpleNamespace(expert_count=6),
        get_many=lambda layer, ids: calls.append((layer, list(ids))) or O.ResidentExperts(
            tuple(experts[e] for e in sorted(set(ids))), {e: i for i, e in enumerate(sorted(set(ids)))}),
        record_routing_sync=lambda s: calls.append(("sync", s >= 0)))
    idx = torch.tensor([[[4, 1], [1, 5]]], dtype=torch.int32)
    table, compact = O.resolve_table(cache, 3, idx)
    assert calls[0] == ("sync", True) and calls[1] == (3, [4, 1, 1, 5])
    assert table.gate_up.shape[0] == 3                      # experts 1, 4, 5
    assert compact.tolist() == [[[1, 0], [0, 2]]]
    assert [int(table.gate_up[i, 0, 0]) for i in range(3)] == [1, 4, 5]


def _pooled_experts(n=6, H=64, I=32):
    """n experts handed out as [i] views of region-major tensors (the reference's get_many,
    expert_cache.py:488-497), each expert's regions filled with its id."""
    gu = torch.arange(n, dtype=torch.int32).repeat_interleave(2 * I * H // 8).reshape(n, 2 * I, H // 8)
    gus = torch.full((n, 2 * I, H // 32), 127, dtype=torch.uint8)
    dn = torch.arange(n, dtype=torch.int32).repeat_interleave(H * I // 8).reshape(n, H, I // 8)
    dns = torch.full((n, H, I // 32), 127, dtype=torch.uint8)
    return [O.QwenExpertWeights(gu[e], gus[e], dn[e], dns[e]) for e in range(n)]


def test_get_many_addresses_pooled_experts_in_place():
    experts = _pooled_experts()
    cache = SimpleNamespace(get_many=lambda _l, ids: O.ResidentExperts(
        tuple(experts[e] for e in sorted(set(ids))), {e: i for i, e in enumerate(sorted(set(ids)))}))
    idx = torch.tensor([[[5, 1], [1, 4]]], dtype=torch.int32)
    table, compact = O.resolve_table(cache, 0, idx)
    # no copy: views from the lowest expert's regions on, and a slot map relative to it
    assert table.slots.tolist() == [0, 3, 4] and table.count == 3
    assert table.gate_up.data_ptr() == experts[1].gate_up.data_ptr()
    assert compact.tolist() == [[[2, 0], [0, 1]]]
    for i, e in enumerate([1, 4, 5]):
        s = int(table.slots[i])
        assert torch.equal(table.gate_up[s], experts[e].gate_up) and torch.equal(table.down[s], experts[e].down)


def test_get_many_copies_experts_outside_one_pool():
    pooled = _pooled_experts(3)
    experts = [pooled[0], _qwen_expert(7), pooled[2]]  # one expert from another allocation
    cache = SimpleNamespace(get_many=lambda _l, ids: O.ResidentExperts(tuple(experts), {0: 0, 1: 1, 2: 2}))
    table, compact = O.resolve_table(cache, 0, torch.tensor([[2, 0, 1]], dtype=torch.int32))
    assert table.slots is None and table.gate_up.shape[0] == 3
    assert [int(table.gate_up[i, 0, 0]) for i in range(3)] == [0, 7, 2]
    assert compact.tolist() == [[2, 0, 1]]


def test_current_batched_needs_no_host_ids_and_records_the_call():
    batched = O.QwenBatchedExperts(*(torch.zeros(4, 2, 2, dtype=d) for d in (torch.int32, torch.uint8,
                                                                            torch.int32, torch.uint8)))
    seen = []
    cache = SimpleNamespace(current_batched=lambda layer: batched, record_gather_qmm=seen.append,
                            route_cache_enabled=True, observe_batched_routes=lambda l, ids: seen.append(ids.shape))
    idx = torch.tensor([[0, 3]], dtype=torch.int32)
    table, same = O.resolve_table(cache, 0, idx, 7.0)
    assert same is idx and table.swiglu_limit == 7.0 and not table.up_first
    assert seen == [(1, 2), 2]


def test_iter_ready_decode_closes_the_iterator():
    experts = {e: _qwen_expert(e) for e in range(4)}
    closed = []

    class Ready:
        def __init__(self, ids):
            self._it = iter([(e, experts[e]) for e in sorted(set(ids), reverse=True)])

        def __iter__(self):
            return self._it

        def close(self):
            closed.append(True)

    cache = SimpleNamespace(ready_expert_decode=True, iter_ready=lambda layer, ids: Ready(ids),
                            get_many=lambda *a: pytest.fail("single-token decode must use iter_ready"))
    table, compact = O.resolve_table(cache, 0, torch.tensor([[2, 0]], dtype=torch.int32))
    assert closed == [True]
    assert compact.tolist() == [[1, 0]] and int(table.gate_up[1, 0, 0]) == 2


def test_out_of_model_ids_raise_value_error():
    cache = SimpleNamespace(model=SimpleNamespace(expert_count=4), get_many=lambda *a: pytest.fail("no acquire"))
    with pytest.raises(ValueError):
        O.resolve_table(cache, 0, torch.tensor([[1, 4]], dtype=torch.int32))
    with pytest.raises(ValueError):
        O.resolve_table(cache, 0, torch.tensor([[-1, 0]], dtype=torch.int32))


def test_missing_resident_expert_raises():
    cache = SimpleNamespace(get_many=lambda layer, ids: O.ResidentExperts((_qwen_expert(0),), {0: 0}))
    with pytest.raises(ValueError):
        O.resolve_table(cache, 0, torch.tensor([[0, 2]], dtype=torch.int32))


def test_activation_descriptors():
    assert O._fused_limit(None) == 0.0
    assert O._fused_limit(O.SwiGLU()) == 0.0
    assert O._fused_limit(O.ClampedSwiGLU(10)) == 10.0
    assert O._fused_limit(lambda up, gate: up) is None
    up = torch.tensor([12.0, -30.0])
    gate = torch.tensor([20.0, 1.0])
    got = O.ClampedSwiGLU(10)(up, gate)
    want = torch.nn.functional.silu(torch.tensor([10.0, 1.0])) * torch.tensor([10.0, -10.0])
    assert torch.allclose(got, want)


def _same_pool(a, b):
    if a is None or b is None:
        return a is None and b is None
    (fa, sa), (fb, sb) = a, b
    return list(sa) == list(sb) and all(
        x.shape == y.shape and x.stride() == y.stride() and x.storage_offset() == y.storage_offset()
        and x.data_ptr() == y.data_ptr() and x.dtype == y.dtype for x, y in zip(fa, fb))


@pytest.mark.skipif(O._host_meta is None, reason="csrc/host_meta.cpp is not built (python -m whallm_amd.build)")
def test_compiled_pool_check_equals_the_python_rules():
    rng = torch.Generator().manual_seed(0)
    experts = _pooled_experts(8)
    regs = lambda ws: [(w.gate_up, w.gate_up_scales, w.down, w.down_scales) for w in ws]  # noqa: E731
    cases = [regs(experts), regs(experts[3:4]), regs([experts[i] for i in (6, 1, 4)])]
    for _ in range(20):  # random subsets in random order
        perm = torch.randperm(8, generator=rng)[:int(torch.randint(1, 9, (1,), generator=rng))]
        cases.append(regs([experts[int(i)] for i in perm]))
    # padded slots: [i, :rows] of a region-major tensor with two spare rows per slot
    pad = torch.zeros(4, 66, 8, dtype=torch.int32)
    padded = [O.QwenExpertWeights(pad[e, :64], experts[e].gate_up_scales, experts[e].down, experts[e].down_scales)
              for e in range(4)]
    cases.append(regs(padded))
    # not one pool: another allocation, a shape or dtype that differs, a repeated expert,
    # a 3-D region, offsets that are not slot multiples of one step
    other = _qwen_expert(7)
    cases.append(regs([experts[0], other]))
    cases.append(regs([experts[0], O.QwenExpertWeights(experts[1].gate_up[:, :4], *regs([experts[1]])[0][1:])]))
    cases.append(regs([experts[0], O.QwenExpertWeights(experts[1].gate_up.view(torch.float32),
                                                       *regs([experts[1]])[0][1:])]))
    cases.append(regs([experts[2], experts[2]]))
    cases.append([(experts[0].gate_up[None], *regs([experts[0]])[0][1:])])
    flat = torch.zeros(1000, dtype=torch.int32)
    odd = [O.QwenExpertWeights(flat[o:o + 64 * 8].view(64, 8), *regs([experts[e]])[0][1:]) for e, o in ((0, 0), (1, 3))]
    cases.append(regs(odd))
    for regs_case in cases:
        assert _same_pool(O._host_meta.pool_regions([t for r in regs_case for t in r], len(regs_case)),
                          O._pool_regions(regs_case))
    assert O._host_meta.pool_regions([], 0) is None
