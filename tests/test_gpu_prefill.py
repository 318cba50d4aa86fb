"""Chunked-prefill scoring on the GPU (MFMA path) against the CPU oracle (R:314-340)."""
from types import SimpleNamespace

import numpy as np
import pytest
import torch

import oracle as O
from fakes import backend, layer

pytestmark = pytest.mark.gpu

ge = None


@pytest.fixture(autouse=True)
def fresh_state():
    global ge
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    import gstar_evict
    ge = gstar_evict
    ge.STATE = None
    yield
    ge.STATE = None


def _case(count, prefix_len, seed, slots=20000):
    g = torch.Generator().manual_seed(seed)
    b = backend(gen=g, slots=slots)
    st = ge.state(b)
    q = (torch.randn((count, 64, 64), generator=g) * 1.5).to(torch.bfloat16).cuda()
    sinks = torch.randn(64, generator=g).to(torch.bfloat16).cuda()
    perm = torch.randperm(slots - 1, generator=g)[:prefix_len + count] + 1
    return b, st, q, sinks, perm[:prefix_len].cuda(), perm[prefix_len:].cuda()


@pytest.mark.parametrize("count,prefix_len,mode,delay", [
    (1, 0, 1, 0), (37, 0, 2, 0), (100, 300, 1, 0), (257, 1000, 2, 0), (130, 64, 1, 0),
    # Score delays (block policies): pass 2 credits keys `delay` positions older than each query
    # only, while pass 1's normaliser covers the whole causal range.
    (257, 1000, 2, 128), (130, 64, 1, 100), (37, 0, 1, 5), (200, 0, 2, 190), (20, 30, 1, 60)])
def test_prefill_scores_match_oracle(count, prefix_len, mode, delay):
    b, st, q, sinks, prefix, new = _case(count, prefix_len, seed=count + prefix_len)
    keys = b.token_to_kv_pool.get_key_buffer(1)
    before = torch.rand(st.scores.shape, generator=torch.Generator().manual_seed(3)).cuda()
    st.scores.copy_(before)
    ge._prefill_scores(st, 0, mode | delay << 8, layer(1), q, keys, sinks, prefix, new)
    upd, slots = O.prefill_score_update(mode, q.float().cpu().numpy(), keys.float().cpu().numpy(),
                                        sinks.float().cpu().numpy(), 0.125, 8, prefix.cpu().numpy(),
                                        new.cpu().numpy(), delay=delay)
    expected = before.clone()
    expected[0][:, torch.tensor(slots).cuda()] += torch.tensor(upd, dtype=torch.float32).cuda()
    torch.testing.assert_close(st.scores, expected, rtol=1e-3, atol=1e-6)


def test_after_extend_scores_chunks_of_two_requests():
    """The hook path: CSR prefix per request, zeroed new slots, sum and max rows in one batch."""
    g = torch.Generator().manual_seed(21)
    b = backend(gen=g)
    st = ge.state(b)
    perm = (torch.randperm(19999, generator=g) + 1).cuda()
    # Request rows 1 (head_sum, prefix 200, 50 new) and 2 (head_max_sum, prefix 0, 70 new).
    pre1, new1 = perm[:200], perm[200:250]
    pre2, new2 = perm[300:300], perm[300:370]
    for row, mode in ((1, 1), (2, 2)):
        st.entries[row] = {"kind": "live", "error": None, "mode": mode}
    q = torch.randn((120, 64, 64), generator=g).to(torch.bfloat16).cuda()
    sinks = torch.randn(64, generator=g).cuda()
    b.forward_metadata = SimpleNamespace(qo_indptr=torch.tensor([0, 50, 120], device="cuda"),
                                         kv_indptr=torch.tensor([0, 200, 200], device="cuda"),
                                         kv_indices=torch.cat((pre1, pre2)))
    fb = SimpleNamespace(req_pool_indices=torch.tensor([1, 2], device="cuda"),
                         out_cache_loc=torch.cat((new1, new2)), extend_prefix_lens_cpu=[200, 0])
    st.scores.fill_(0.5)
    ge.after_extend(b, q.reshape(120, -1), layer(1), fb, sinks)
    keys = b.token_to_kv_pool.get_key_buffer(1).float().cpu().numpy()
    expected = torch.full_like(st.scores, 0.5)
    expected[:, :, torch.cat((new1, new2))] = 0.0
    for (pre, new, lo, hi, mode) in ((pre1, new1, 0, 50, 1), (pre2, new2, 50, 120, 2)):
        upd, slots = O.prefill_score_update(mode, q[lo:hi].float().cpu().numpy(), keys, sinks.cpu().numpy(), 0.125,
                                            8, pre.cpu().numpy(), new.cpu().numpy())
        expected[0][:, torch.tensor(slots).cuda()] += torch.tensor(upd, dtype=torch.float32).cuda()
    torch.testing.assert_close(st.scores, expected, rtol=1e-3, atol=1e-6)


def test_prefill_mass_is_conserved_at_8k_chunk():
    """A full 8192-query chunk after a 2048-key prefix: head-sum scores of a KV head add up to the
    non-sink probability mass of its 8 query heads over all queries (a size-independent check)."""
    count, prefix_len = 8192, 2048
    b, st, q, sinks, prefix, new = _case(count, prefix_len, seed=5, slots=12000)
    keys = b.token_to_kv_pool.get_key_buffer(1)
    st.scores.zero_()
    ge._prefill_scores(st, 0, 1, layer(1), q, keys, sinks, prefix, new)
    got = st.scores[0].double().sum(1)  # [kv head]
    # Sink mass per (query, head) from the oracle on a sample of queries, exact elsewhere by sum.
    kk = keys[torch.cat((prefix, new))].float()
    total = torch.zeros(8, dtype=torch.float64)
    for lo in range(0, count, 1024):
        hi = lo + 1024
        qq = q[lo:hi].float().view(hi - lo, 8, 8, 64)
        logits = torch.einsum("qgjd,kgd->gjqk", qq, kk) * 0.125
        pos = prefix_len + torch.arange(lo, hi, device="cuda")
        logits.masked_fill_(torch.arange(kk.shape[0], device="cuda")[None, None, None, :] > pos[None, None, :, None],
                            -torch.inf)
        lse = torch.logsumexp(logits, -1)
        norm = torch.logaddexp(lse, sinks.float().view(8, 8, 1))
        sink_p = torch.exp(sinks.float().view(8, 8, 1) - norm)
        total += (1 - sink_p).sum((1, 2)).double().cpu()
    torch.testing.assert_close(got.cpu(), total, rtol=1e-4, atol=1e-3)
