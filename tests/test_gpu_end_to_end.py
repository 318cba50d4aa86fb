"""The reference's CPU-runnable case end to end, through the hooks SGLang calls.

One full-attention layer (64 query heads, 8 KV heads, d=64), Q/K/V ~ N(0, 1) from seed 0,
scale 1/sqrt(64), sink logits ~ N(0, 1). A 4096-token prompt arrives in two 2048-token
chunks (`on_extend` + `after_extend`), then decode steps run `on_decode`, `fill` and the
fused `decode`; the boundary at 4096 fires at the first decode step with head_sum at budget
2048 = 128 prefix + 512 recent + 1408 scored. `on_decode` queues it and the next `on_decode`
does its host part, so the device state is checked in between and the entry after. Every stage is compared with the oracle: prefill
scores, the boundary's retained positions, table, req_to_token, relocated K/V/scores and freed
slots (bit-exact, the oracle ranking the GPU's own pre-boundary scores), each step's attention
output, and the accumulated scores after the last step.

The block policies (no reference counterpart) run the same flow with a score delay of 128
positions, which the oracle applies by position (a query credits keys at least 128 positions
older) and the kernels by cutting each list's last 128 entries: equal scores show that every
list ends with its newest positions in order, before and after the boundary. One of them caps
the evicted blocks so that the boundary keeps more than the budget (3072 of 2048).
"""
import sys
import types
from types import SimpleNamespace

import numpy as np
import pytest
import torch

import oracle as O
from fakes import allocator, backend, layer

pytestmark = pytest.mark.gpu

PROMPT, CHUNK, STEPS = 4096, 2048, 256
BUDGET, PREFIX, RECENT = 2048, 128, 512
SCALE = 0.125
ROW = 1


@pytest.fixture(autouse=True)
def fake_sglang(monkeypatch):
    """The one SGLang import the hooks make (the SWA component id)."""
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    names = ["sglang", "sglang.srt", "sglang.srt.mem_cache", "sglang.srt.mem_cache.unified_cache",
             "sglang.srt.mem_cache.unified_cache.component_type"]
    for name in names:
        monkeypatch.setitem(sys.modules, name, types.ModuleType(name))
    sys.modules[names[-1]].ComponentType = SimpleNamespace(SWA="swa")
    import gstar_evict
    gstar_evict.STATE = None
    yield gstar_evict
    gstar_evict.STATE = None


def _request(cfg, lengths):
    """A request whose SWA cursor trails its current length by 128 tokens (gpt-oss's window)."""
    req = SimpleNamespace(rid="r0", session=None, retraction_count=0,
                          sampling_params=SimpleNamespace(custom_params={"gstar_eviction": cfg}))
    req.kv = SimpleNamespace(req_pool_idx=ROW, get_evicted_seqlen=lambda kind: max(lengths[0] - 128, 0))
    return req


def _assert_same_positions(got, want, scores, slot_of):
    """Retained positions equal; on a mismatch, name a head and the scores of what differs."""
    if np.array_equal(got, want):
        return
    for g in range(got.shape[1]):
        a, c = set(got[0, g].tolist()), set(want[0, g].tolist())
        if a != c:
            only_gpu, only_oracle = sorted(a - c)[:8], sorted(c - a)[:8]
            sc = scores[0, g]
            raise AssertionError(f"head {g}: kept only by the GPU {only_gpu} (scores "
                                 f"{[float(sc[slot_of[x]]) for x in only_gpu]}), only by the oracle "
                                 f"{only_oracle} (scores {[float(sc[slot_of[x]]) for x in only_oracle]})")
    raise AssertionError("retained positions differ in order only")


CONFIGS = {
    "head_sum": ({"name": "head_sum_2048"}, BUDGET),
    # 16-token layer-shared blocks, delay 128, at most 64 blocks evicted: the boundary at 4096 keeps
    # 4096 - 64 * 16 = 3072 columns.
    "block_sum_capped": ({"name": "block_sum_2048", "block": 16, "shared": True, "score_delay": 128,
                          "max_evicted_blocks": 64}, 3072),
    # The reference report's settings: 4-token blocks scored by their maximum, delay 128, cap 512.
    "block_max_report": ({"name": "block_max_2048", "block": 4, "shared": True, "score_delay": 128,
                          "max_evicted_blocks": 512}, BUDGET),
    # The same settings with the report's block score (TEX:197): per-block counters, each query
    # adding the maximum over a whole, 128-position-old block's keys and all 64 query heads.
    "block_counters_report": ({"name": "block_max_2048", "block": 4, "shared": True, "score_delay": 128,
                               "max_evicted_blocks": 512, "block_score": "step_max"}, BUDGET),
}


@pytest.mark.parametrize("case", list(CONFIGS))
def test_prompt_boundary_and_decode_match_the_oracle(fake_sglang, case):
    ge = fake_sglang
    g = torch.Generator().manual_seed(0)
    slots_total = PROMPT + STEPS + 64
    b = backend(rows=2, width=8192, slots=slots_total, layers=1, full=(0,), gen=g)
    freed, alloc = allocator(slots=slots_total)
    st = ge.state(b)
    st.score_mode = "queue"
    lay = layer(0, scaling=SCALE)
    q_all = torch.randn((PROMPT + STEPS, 64, 64), generator=g).to(torch.bfloat16).cuda()
    sinks = torch.randn(64, generator=g).to(torch.bfloat16).cuda()
    slot_of = (torch.randperm(slots_total - 1, generator=g)[:PROMPT + STEPS] + 1).cuda()
    keys, values = b.token_to_kv_pool.get_key_buffer(0), b.token_to_kv_pool.get_value_buffer(0)

    extra, kept = CONFIGS[case]
    cfg = {"budget": BUDGET, "prefix": PREFIX, "recent": RECENT, "seed": 0, **extra}
    delay = cfg.get("score_delay", 0)
    lengths = [0]
    req = _request(cfg, lengths)
    batch = SimpleNamespace(reqs=[req], tree_cache=SimpleNamespace(token_to_kv_pool_allocator=alloc))

    ost = O.OracleState([keys.float().cpu().numpy()], [values.float().cpu().numpy()],
                        st.req_to_token.cpu().numpy())
    oe = O.live_entry(cfg)
    mode = oe["mode"]
    kn, sn = ost.keys[0], sinks.float().cpu().numpy()
    rows = torch.tensor([ROW], device="cuda")

    # Prompt: two chunks; the chunk at 2048 triggers a boundary with nothing to evict.
    for start in range(0, PROMPT, CHUNK):
        new = slot_of[start:start + CHUNK]
        st.req_to_token[ROW, start:start + CHUNK] = new.int()
        ost.req_to_token[ROW, start:start + CHUNK] = new.cpu().numpy()
        lengths[0] = start
        req.extend_range = SimpleNamespace(start=start, length=CHUNK)
        ge.on_extend(batch)
        if start:
            ofreed = []
            O.boundary(ost, ROW, oe, start, start - 128, free=ofreed.append)
        prefix = torch.zeros(start + 1, dtype=torch.int32, device="cuda")
        b.kv_indptr.zero_()
        ge.fill(b, 1, torch.tensor([start], device="cuda"), rows, prefix)
        b.forward_metadata = SimpleNamespace(qo_indptr=torch.tensor([0, CHUNK], device="cuda"),
                                             kv_indptr=b.kv_indptr[:2].clone(), kv_indices=prefix[:start])
        fb = SimpleNamespace(req_pool_indices=rows, out_cache_loc=new, extend_prefix_lens_cpu=[start])
        ge.after_extend(b, q_all[start:start + CHUNK].reshape(CHUNK, -1), lay, fb, sinks)
        # Oracle chunk scores, 256 queries at a time (the probability tile stays small).
        pre = slot_of[:start].cpu().numpy()
        for lo in range(0, CHUNK, 256):
            chunk_q = q_all[start + lo:start + lo + 256].float().cpu().numpy()
            seen = np.concatenate((pre, new[:lo].cpu().numpy()))
            if mode == O.BLOCK_STEP:
                upd, sl = O.prefill_block_step_update(chunk_q, kn, sn, SCALE, 8, seen, new[lo:lo + 256].cpu().numpy(),
                                                      cfg["block"], delay=delay)
                ost.scores[0][0, sl] += upd.astype(np.float32)
                continue
            upd, sl = O.prefill_score_update(mode, chunk_q, kn, sn, SCALE, 8, seen, new[lo:lo + 256].cpu().numpy(),
                                             delay=delay)
            ost.scores[0][:, sl] += upd.astype(np.float32)
    entry = st.entries[ROW]
    assert [ev["after"] for ev in entry["events"]] == [CHUNK] == [ev["after"] for ev in oe["events"]]
    torch.testing.assert_close(st.scores.cpu(), torch.tensor(ost.scores), rtol=2e-3, atol=1e-6)

    outs, want_outs = [], []
    for t in range(STEPS):
        p = PROMPT + t
        lengths[0] = p
        if t == 0:
            # The oracle ranks the GPU's own pre-boundary scores, so selection compares bit-exactly.
            ost.scores = st.scores.cpu().numpy().copy()
            pre_scores = ost.scores.copy()
        ge.on_decode(SimpleNamespace(reqs=[req], seq_lens_cpu=torch.tensor([p]),
                                     tree_cache=SimpleNamespace(token_to_kv_pool_allocator=alloc)))
        if t == 0:
            # The boundary is queued, its host part pending: the device state is already its
            # outcome, the entry and the allocator are not yet.
            ofreed = []
            O.boundary(ost, ROW, oe, p, p - 128, free=ofreed.append)
            assert len(st.pending) == 1 and entry["count"] == 0 and not freed
            assert oe["count"] == kept
            assert np.array_equal(st.table[ROW, :kept].cpu().numpy(), ost.table[ROW, :kept])
            assert np.array_equal(st.req_to_token[ROW].cpu().numpy(), ost.req_to_token[ROW])
            assert int(st.count[ROW]) == kept and int(st.frontier[ROW]) == p
            assert np.array_equal(keys.float().cpu().numpy(), ost.keys[0])
            assert np.array_equal(values.float().cpu().numpy(), ost.values[0])
            assert np.array_equal(st.scores.cpu().numpy(), ost.scores)
        if t == 1:
            # The next decode hook finished it.
            assert not st.pending
            assert entry["count"] == oe["count"] == kept and entry["frontier"] == PROMPT
            _assert_same_positions(entry["pos"].cpu().numpy(), oe["pos"], pre_scores, slot_of.cpu().numpy())
            assert np.array_equal(torch.cat(freed).cpu().numpy(), ofreed[0])
            assert [ev["after"] for ev in entry["events"]][-1] == kept
        # SGLang's allocation of the new token, then the CSR and the fused decode.
        new = slot_of[p:p + 1]
        st.req_to_token[ROW, p] = new.int()
        ost.req_to_token[ROW, p] = int(new)
        kv_indices = torch.zeros(p + 1, dtype=torch.int32, device="cuda")
        ge.fill(b, 1, torch.tensor([p + 1], device="cuda"), rows, kv_indices)
        b.forward_metadata = SimpleNamespace(kv_indptr=b.kv_indptr[:2], kv_indices=kv_indices)
        fb = SimpleNamespace(out_cache_loc=new, req_pool_indices=rows, seq_lens_cpu=torch.tensor([p + 1]))
        o = torch.empty((1, 64, 64), dtype=torch.bfloat16, device="cuda")
        assert ge.decode(b, q_all[p:p + 1].reshape(1, -1), lay, fb, sinks, o.reshape(1, -1))
        outs.append(o[0])
        # Oracle step: the resident list is the table then the tail (R:136-152).
        res = np.concatenate((ost.table[ROW, :oe["count"]], ost.req_to_token[ROW, oe["frontier"]:p + 1]))
        qn = q_all[p].float().cpu().numpy()
        want_o, norm = O.decode_attention(qn, ost.keys[0], ost.values[0], res, sn, SCALE)
        ost.scores[:, :, int(new)] = 0.0
        key_pos = np.arange(p + 1)
        if oe["count"]:
            tail = np.arange(oe["frontier"], p + 1)
            key_pos = np.concatenate((oe["pos"][0], np.broadcast_to(tail, (8, tail.size))), axis=1)
        if mode == O.BLOCK_STEP:  # shared blocks: every KV head holds the same positions
            O.decode_block_step_into(ost.scores[0], qn, ost.keys[0], res, norm, SCALE, cfg["block"],
                                     key_pos if key_pos.ndim == 1 else key_pos[0], p, delay)
        else:
            O.decode_scores_into(ost.scores[0], qn, ost.keys[0], res, norm, SCALE, mode, key_pos, p, delay)
        want_outs.append(want_o)
    ge.flush(st)
    got = torch.stack(outs).float().cpu().numpy()
    want = np.stack(want_outs)
    np.testing.assert_allclose(got, want, rtol=2e-2, atol=2e-2)
    assert np.abs(got - want).mean() < 2e-3
    torch.testing.assert_close(st.scores.cpu(), torch.tensor(ost.scores), rtol=2e-3, atol=1e-6)
    if mode == O.BLOCK_STEP:
        # Counters sit in KV head 0 at the first slot of each whole, credited block only.
        assert float(st.scores[0, 1:].abs().sum()) == 0.0
        held = np.concatenate((entry["pos"][0, 0].cpu().numpy(), np.arange(entry["frontier"], PROMPT + STEPS)))
        listed = np.concatenate((st.table[ROW, :entry["count"]].cpu().numpy(),
                                 st.req_to_token[ROW, entry["frontier"]:PROMPT + STEPS].cpu().numpy()))
        nonzero = st.scores[0, 0, torch.tensor(listed, device="cuda").long()].cpu().numpy() != 0
        assert np.all(held[nonzero] % cfg["block"] == 0) and nonzero.sum() > 400  # of 576 blocks
