"""Static replay's layer difference on the GPU (R:520-546) against the oracle.

At gpt-oss shape (64 query heads, 8 KV heads, d=64): K/V ~ N(0, 1) with 2% planted heavy keys
(norm x4 along a per-head direction the queries share), so evicting them moves real attention
mass. Errors agree with the float64 oracle to rtol 1e-3 + atol 1e-5 (the kernel's logits are
fp32 sums of exact bf16 products; probabilities enter the value product as bf16 hi + lo).
"""
import sys
import types
from types import SimpleNamespace

import numpy as np
import pytest
import torch

import oracle as O
from fakes import FULL, backend, layer

pytestmark = pytest.mark.gpu

HEADS, KV_HEADS, DIM = 64, 8, 64
RTOL, ATOL = 1e-3, 1e-5


@pytest.fixture(autouse=True)
def runtime():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    import gstar_evict
    gstar_evict.STATE = None
    yield gstar_evict
    gstar_evict.STATE = None


def _shadow(rows, gen):
    """Shadow K/V [rows, 8, 64] bf16 with 2% heavy keys along a per-head direction; the queries
    lean on the same directions."""
    k = torch.randn((rows, KV_HEADS, DIM), generator=gen)
    v = torch.randn((rows, KV_HEADS, DIM), generator=gen)
    direction = torch.nn.functional.normalize(torch.randn((KV_HEADS, DIM), generator=gen), dim=-1)
    heavy = torch.rand((rows, KV_HEADS), generator=gen) < 0.02
    k = torch.where(heavy[..., None], 4 * k.norm(dim=-1, keepdim=True) * direction, k)
    return k.to(torch.bfloat16), v.to(torch.bfloat16), direction


def _queries(count, direction, gen):
    q = torch.randn((count, HEADS, DIM), generator=gen) + 1.5 * direction.repeat_interleave(HEADS // KV_HEADS, 0)
    return q.to(torch.bfloat16)


def _retained(frontier, kept, gen, stride=None):
    """Per KV head, `kept` sorted positions below the frontier as int32 [1, 8, kept] (a view of
    a [1, 8, stride] buffer when stride is given, as the boundary leaves it)."""
    pos = torch.stack([torch.randperm(frontier, generator=gen)[:kept].sort().values for _ in range(KV_HEADS)])
    buf = torch.zeros((1, KV_HEADS, stride or kept), dtype=torch.int32)
    buf[0, :, :kept] = pos.int()
    return buf.cuda()[..., :kept]


def _run(ge, q, k, v, sinks, entry, start):
    st = ge.state(backend(rows=2, width=64, slots=16, layers=2, full=(1,)))
    entry = dict(entry, shadow_k=k.cuda(), shadow_v=v.cuda(), layer_error=[])
    ge._replay_layer_difference(st, entry, q.cuda(), layer(1), sinks.cuda(), start)
    torch.cuda.synchronize()
    return entry["layer_error"][0].cpu().numpy()


def _oracle(q, k, v, sinks, entry, start):
    end = start + q.shape[0]
    pos = {"frontier": entry["frontier"], "count": entry["count"],
           "pos": entry["pos"].cpu().numpy() if entry["count"] else None}
    visible = O.visible_positions(pos, end, KV_HEADS)
    return O.replay_layer_difference(q.float().numpy(), k.float().numpy(), v.float().numpy(), sinks.float().numpy(),
                                     0.125, KV_HEADS, visible, start)


@pytest.mark.parametrize("start,count,frontier,kept,stride", [
    (2048, 512, 2048, 700, None),     # the chunk right after a boundary
    (2560, 77, 2048, 300, 1024),      # a later, ragged chunk; the retained rows are a strided view
    (4096, 256, 4096, 2048, None),    # budget-sized retention
])
def test_layer_difference_matches_the_oracle(runtime, start, count, frontier, kept, stride):
    gen = torch.Generator().manual_seed(start + count)
    k, v, direction = _shadow(start + count + 5, gen)
    q = _queries(count, direction, gen)
    sinks = torch.randn(HEADS, generator=gen)
    entry = {"frontier": frontier, "count": kept, "pos": _retained(frontier, kept, gen, stride)}
    print(f"replay start={start} count={count} frontier={frontier} kept={kept}", flush=True)
    got = _run(runtime, q, k, v, sinks, entry, start)
    want = _oracle(q, k, v, sinks, entry, start)
    assert want.min() > 1e-3  # evicting heavy keys moves the output
    np.testing.assert_allclose(got, want, rtol=RTOL, atol=ATOL)


def test_layer_difference_is_zero_before_any_eviction(runtime):
    gen = torch.Generator().manual_seed(9)
    k, v, direction = _shadow(700, gen)
    q = _queries(300, direction, gen)
    got = _run(runtime, q, k, v, torch.randn(HEADS, generator=gen), {"frontier": 0, "count": 0, "pos": None}, 400)
    assert np.array_equal(got, np.zeros(300, dtype=np.float32))


def test_small_differences_are_resolved(runtime):
    """Flat attention over values with a shared mean, 32 of 2048 old keys evicted: errors of
    ~5e-4 still agree with the oracle to 1e-5, which needs the probabilities' low bits in the
    value product (bf16 probabilities alone are off by ~4e-5 here)."""
    gen = torch.Generator().manual_seed(4)
    start, count, frontier = 2048, 128, 2048
    k = (torch.randn((start + count, KV_HEADS, DIM), generator=gen) * 0.3).to(torch.bfloat16)
    v = (1 + 0.2 * torch.randn((start + count, KV_HEADS, DIM), generator=gen)).to(torch.bfloat16)
    q = torch.randn((count, HEADS, DIM), generator=gen).to(torch.bfloat16)
    sinks = torch.randn(HEADS, generator=gen)
    entry = {"frontier": frontier, "count": frontier - 32, "pos": _retained(frontier, frontier - 32, gen)}
    got = _run(runtime, q, k, v, sinks, entry, start)
    want = _oracle(q, k, v, sinks, entry, start)
    assert want.max() < 2e-3
    np.testing.assert_allclose(got, want, rtol=RTOL, atol=ATOL)


def test_entry_point_validation(runtime):
    from gstar_evict import _native as N
    ws = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")
    err = torch.empty(4, device="cuda")
    q = torch.zeros((4, HEADS, DIM), dtype=torch.bfloat16, device="cuda")
    kv = torch.zeros((16, KV_HEADS, DIM), dtype=torch.bfloat16, device="cuda")
    pos = torch.zeros((KV_HEADS, 4), dtype=torch.int32, device="cuda")
    sinks = torch.zeros(HEADS, device="cuda")

    def call(start=8, rows=16, frontier=8, retained_count=4, heads=HEADS, ws_bytes=ws.numel()):
        return N.lib().gse_replay_layer_difference(
            N.ptr(q), HEADS * DIM, DIM, 4, N.ptr(kv), N.ptr(kv), KV_HEADS * DIM, DIM, rows, start, N.ptr(pos), 4,
            retained_count, frontier, N.ptr(sinks), N.float_code(sinks), heads, KV_HEADS, DIM, 0.125, N.ptr(err),
            N.ptr(ws), ws_bytes, N.stream())

    assert call() == 0
    assert call(frontier=9) != 0  # the chunk starts before the frontier
    assert call(rows=11) != 0  # the shadow does not reach the chunk's end
    assert call(heads=32) != 0
    assert call(ws_bytes=1024) != 0
    torch.cuda.synchronize()


def test_hooks_write_the_replay_payload(runtime, tmp_path, monkeypatch):
    """`gstar_replay` through the hooks: the boundary at 2048 relocates without freeing, the
    next chunk's first-full-layer errors reach the payload's layer_error (R:732-736)."""
    from gstar_evict import retention
    ge = runtime
    monkeypatch.setenv("GSTAR_PAYLOAD_DIR", str(tmp_path))
    names = ["sglang", "sglang.srt", "sglang.srt.mem_cache", "sglang.srt.mem_cache.unified_cache",
             "sglang.srt.mem_cache.unified_cache.component_type"]
    for name in names:
        monkeypatch.setitem(sys.modules, name, types.ModuleType(name))
    sys.modules[names[-1]].ComponentType = SimpleNamespace(SWA="swa")
    length, row = 2048 + 300, 1
    g = torch.Generator().manual_seed(12)
    b = backend(rows=2, width=length + 8, slots=length + 8, gen=g)
    st = ge.state(b)
    cfg = {"name": "head_sum_2048", "budget": 1024, "prefix": 64, "recent": 256, "seed": 0}
    req = SimpleNamespace(rid="rep1", session=None, retraction_count=0, origin_input_ids=[0] * length,
                          sampling_params=SimpleNamespace(custom_params={"gstar_replay": cfg}),
                          kv=SimpleNamespace(req_pool_idx=row, holds_kv=True, get_evicted_seqlen=lambda kind: 0))
    batch = SimpleNamespace(reqs=[req], tree_cache=SimpleNamespace(token_to_kv_pool_allocator=None))
    slot_of = torch.arange(1, length + 1, device="cuda")
    st.req_to_token[row, :length] = slot_of.int()
    rows = torch.tensor([row], device="cuda")
    first = FULL[0]
    keys = b.token_to_kv_pool.get_key_buffer(first)[1:length + 1].cpu()
    values = b.token_to_kv_pool.get_value_buffer(first)[1:length + 1].cpu()
    sinks = torch.randn(HEADS, generator=g)
    chunk_q = {}
    for lo, hi in ((0, 2048), (2048, length)):
        req.extend_range = SimpleNamespace(start=lo, length=hi - lo)
        ge.on_extend(batch)
        b.forward_metadata = SimpleNamespace(qo_indptr=torch.tensor([0, hi - lo], device="cuda"),
                                             kv_indptr=torch.tensor([0, lo], device="cuda", dtype=torch.int32),
                                             kv_indices=slot_of[:lo].int())
        fb = SimpleNamespace(req_pool_indices=rows, out_cache_loc=slot_of[lo:hi], extend_prefix_lens_cpu=[lo])
        for lid in FULL:
            q = torch.randn((hi - lo, HEADS, DIM), generator=g).to(torch.bfloat16)
            if lid == first:
                chunk_q[lo] = q
            ge.after_extend(b, q.cuda().reshape(hi - lo, -1), layer(lid), fb, sinks.cuda())
    entry = st.entries[row]
    assert entry["kind"] == "replay" and entry["error"] is None
    assert entry["count"] == 1024 and entry["frontier"] == 2048
    retained = {"frontier": 2048, "count": 1024, "pos": entry["pos"][:1].cpu().numpy()}
    ge.release(req)
    payload = retention.read_payload(tmp_path / "rep1.json.gz")
    assert payload["kind"] == "replay" and payload["layer"] == first
    err = payload["layer_error"]
    assert err.shape == (length,) and err.dtype == np.float32
    assert np.array_equal(err[:2048], np.zeros(2048, dtype=np.float32))
    visible = O.visible_positions(retained, length, KV_HEADS)
    want = O.replay_layer_difference(chunk_q[2048].float().numpy(), keys.float().numpy(), values.float().numpy(),
                                     sinks.numpy(), 0.125, KV_HEADS, visible, 2048)
    np.testing.assert_allclose(err[2048:], want, rtol=RTOL, atol=ATOL)
