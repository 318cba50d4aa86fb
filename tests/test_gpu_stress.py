"""Eviction at every decode step with exact-duplicate keys (the radix select's tie case), at a
size the oracle runs in seconds: two rows, two full layers, budget 512 = 64 prefix + 128
recent + 320 scored, 1024-token starting lengths, near-uniform scores and 10 % of each full
layer's keys copied from other slots (their scores copied too, so the duplicates stay exactly
tied through every score update).

Each step: flush the queued scores, compare them with the oracle's update of the previous
step, let the oracle rank exactly the GPU's scores, run both boundaries and compare the state
bit-exactly, then one fused decode step per full layer against the oracle's attention output.
"""
from types import SimpleNamespace

import numpy as np
import pytest
import torch

import oracle as O
from fakes import FULL, allocator, backend, entry, layer

pytestmark = pytest.mark.gpu

ROWS, START, STEPS = (1, 2), 1024, 24
BUDGET, PREFIX, RECENT = 512, 64, 128
SLOTS = 4096


@pytest.fixture(autouse=True)
def fresh_state():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    import gstar_evict
    gstar_evict.STATE = None
    yield gstar_evict
    gstar_evict.STATE = None


def _oracle_state(b, st):
    keys = [b.token_to_kv_pool.get_key_buffer(l).float().cpu().numpy() for l in FULL]
    values = [b.token_to_kv_pool.get_value_buffer(l).float().cpu().numpy() for l in FULL]
    return O.OracleState(keys, values, st.req_to_token.cpu().numpy(), st.scores.cpu().numpy())


@pytest.mark.parametrize("name", ["head_sum_2048", "head_max_sum_2048"])
def test_eviction_every_step_with_exact_duplicate_keys(fresh_state, name):
    ge = fresh_state
    g = torch.Generator().manual_seed(11)
    b = backend(rows=3, width=2048, slots=SLOTS, gen=g)
    st = ge.state(b)
    st.score_mode = "queue"
    perm = (torch.randperm(SLOTS - 1, generator=g) + 1).cuda()
    slot_of = {row: perm[i * (START + STEPS):(i + 1) * (START + STEPS)] for i, row in enumerate(ROWS)}
    # 10 % exact duplicates: K rows (all heads) and scores copied from other slots of the same layer.
    scores0 = torch.rand(st.scores.shape, generator=g).cuda() * 1e-3 + 1.0
    for index, lid in enumerate(FULL):
        k = b.token_to_kv_pool.get_key_buffer(lid)
        dst = perm[torch.randperm(perm.numel(), generator=g)[:perm.numel() // 10].cuda()]
        src = perm[torch.randint(0, perm.numel(), (dst.numel(),), generator=g).cuda()]
        k[dst] = k[src]
        scores0[index][:, dst] = scores0[index][:, src]
    st.scores.copy_(scores0)
    freed, alloc = allocator(slots=SLOTS)
    lens = {}
    entries, oentries = {}, {}
    for row in ROWS:
        st.req_to_token[row, :START] = slot_of[row][:START].int()
        e = entry(ge, name, BUDGET, PREFIX, RECENT, seed=0)
        st.entries[row] = e
        st.mode[row] = e["mode"]
        entries[row], oentries[row] = e, O.live_entry(dict(e["cfg"]))
        lens[row] = START
    ost = _oracle_state(b, st)
    rows_t = torch.tensor(ROWS, device="cuda")
    q_all = torch.randn((STEPS, len(ROWS), 64, 64), generator=g).to(torch.bfloat16).cuda()
    sinks = {lid: torch.randn(64, generator=g).to(torch.bfloat16).cuda() for lid in FULL}
    mode = 1 if name == "head_sum_2048" else 2
    ties_seen = 0
    for t in range(STEPS):
        ge.flush(st)
        got = st.scores.cpu().numpy()
        if t:
            np.testing.assert_allclose(got, ost.scores, rtol=2e-3, atol=1e-6)
        ost.scores = got.copy()
        for row in ROWS:
            n = lens[row]
            e, oe = entries[row], oentries[row]
            before = oe["count"] + n - oe["frontier"]
            slots = np.concatenate((ost.table[row, :oe["count"]], ost.req_to_token[row, oe["frontier"]:n]))
            ties_seen += before - np.unique(ost.scores[0][0, slots]).size
            ofreed = []
            ge._boundary(st, row, e, n, None, alloc)
            O.boundary(ost, row, oe, n, None, free=ofreed.append)
            assert e["count"] == oe["count"] == BUDGET, (t, row)
            assert np.array_equal(e["pos"].cpu().numpy(), oe["pos"]), (t, row)
            assert np.array_equal(st.table[row, :BUDGET].cpu().numpy(), ost.table[row, :BUDGET]), (t, row)
            assert np.array_equal(torch.cat(freed[-1:]).cpu().numpy(), ofreed[0]), (t, row)
        assert np.array_equal(st.req_to_token.cpu().numpy(), ost.req_to_token)
        assert np.array_equal(st.scores.cpu().numpy(), ost.scores)
        for index, lid in enumerate(FULL):
            assert np.array_equal(b.token_to_kv_pool.get_key_buffer(lid).float().cpu().numpy(), ost.keys[index])
            assert np.array_equal(b.token_to_kv_pool.get_value_buffer(lid).float().cpu().numpy(), ost.values[index])
        # One decode step: SGLang's new slot per row, the CSR, the fused kernel per full layer.
        new = torch.stack([slot_of[row][lens[row]] for row in ROWS])
        for i, row in enumerate(ROWS):
            st.req_to_token[row, lens[row]] = new[i].int()
            ost.req_to_token[row, lens[row]] = int(new[i])
            lens[row] += 1
        ge.begin_decode_step(list(ROWS), st)
        seq = torch.tensor([lens[row] for row in ROWS], device="cuda")
        kv_indices = torch.zeros(sum(lens.values()), dtype=torch.int32, device="cuda")
        ge.fill(b, len(ROWS), seq, rows_t, kv_indices)
        b.forward_metadata = SimpleNamespace(kv_indptr=b.kv_indptr[:len(ROWS) + 1], kv_indices=kv_indices)
        fb = SimpleNamespace(out_cache_loc=new, req_pool_indices=rows_t, seq_lens_cpu=seq.cpu())
        ost.scores[:, :, new.cpu().numpy()] = 0.0
        for index, lid in enumerate(FULL):
            o = torch.empty((len(ROWS), 64, 64), dtype=torch.bfloat16, device="cuda")
            assert ge.decode(b, q_all[t].reshape(len(ROWS), -1), layer(lid), fb, sinks[lid], o.reshape(len(ROWS), -1))
            for i, row in enumerate(ROWS):
                oe = oentries[row]
                res = np.concatenate((ost.table[row, :oe["count"]], ost.req_to_token[row, oe["frontier"]:lens[row]]))
                qn = q_all[t, i].float().cpu().numpy()
                want_o, norm = O.decode_attention(qn, ost.keys[index], ost.values[index], res,
                                                  sinks[lid].float().cpu().numpy(), 0.125)
                np.testing.assert_allclose(o[i].float().cpu().numpy(), want_o, rtol=2e-2, atol=2e-2)
                O.decode_scores_into(ost.scores[index], qn, ost.keys[index], res, norm, 0.125, mode)
    assert ties_seen > 0, "the duplicate keys produced no exact score ties"
