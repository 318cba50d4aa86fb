"""Block counters (score kind 4) on the GPU against the oracle: the reference report's block score
(TEX:197; no reference code), where each query adds to every whole block at least `delay`
positions old the maximum over the block's keys and all 64 query heads of its probability, kept in
KV head 0's score of the block's first slot. Decode (eager and queued), prefill chunks, and lists
after block evictions (kept whole blocks, then the tail)."""
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


def word(block, delay):
    return 4 | (block.bit_length() - 1) << 4 | delay << 8


def _numpy(t):
    return t.float().cpu().numpy()


def _decode(b, st, q, sinks, lists, rows, queued, block, delay):
    """One decode step of the rows (their lists given as slot tensors) through the hook."""
    st.score_mode = "queue" if queued else "eager"
    for r in rows:
        st.mode[r] = word(block, delay)
        st.entries[r] = {"mode": 4}  # the flush routes kind-4 rows to their own kernel
    lens = [int(x.numel()) for x in lists]
    indptr = torch.tensor(np.concatenate(([0], np.cumsum(lens))), dtype=torch.int32, device="cuda")
    b.forward_metadata = SimpleNamespace(kv_indptr=indptr, kv_indices=torch.cat(lists))
    fb = SimpleNamespace(out_cache_loc=torch.zeros(len(rows), dtype=torch.int64, device="cuda"),
                         req_pool_indices=torch.tensor(rows, device="cuda"), seq_lens_cpu=torch.tensor(lens))
    o = torch.empty_like(q)
    assert ge.decode(b, q.reshape(len(rows), -1), layer(1), fb, sinks, o.reshape(len(rows), -1))


def _oracle_counters(b, q, sinks, lists, positions, queries_at, block, delay, scores=None):
    keys, values = _numpy(b.token_to_kv_pool.get_key_buffer(1)), _numpy(b.token_to_kv_pool.get_value_buffer(1))
    scores = np.zeros((8, keys.shape[0])) if scores is None else scores
    for i, slots in enumerate(lists):
        sl = slots.cpu().numpy()
        qn = _numpy(q[i])
        _, norm = O.decode_attention(qn, keys, values, sl, _numpy(sinks), 0.125)
        O.decode_block_step_into(scores, qn, keys, sl, norm, 0.125, block, positions[i], queries_at[i], delay)
    return scores


@pytest.mark.parametrize("queued", [False, True])
@pytest.mark.parametrize("block,delay", [(4, 0), (4, 128), (64, 100), (1, 0), (16, 7)])
def test_decode_block_counters_match_the_oracle(queued, block, delay):
    """Fresh lists (positions 0..len-1) of 37, 1500 and 3001 keys; the 37-key list credits nothing
    at delay 100 and above."""
    g = torch.Generator().manual_seed(block + delay)
    b = backend(gen=g, slots=20000, rows=4)
    st = ge.state(b)
    lengths = [37, 1500, 3001]
    q = torch.randn((3, 64, 64), generator=g).to(torch.bfloat16).cuda()
    sinks = torch.randn(64, generator=g).to(torch.bfloat16).cuda()
    perm = (torch.randperm(19999, generator=g)[:sum(lengths)] + 1).cuda()
    cuts = np.concatenate(([0], np.cumsum(lengths)))
    lists = [perm[cuts[i]:cuts[i + 1]] for i in range(3)]
    rows = [1, 2, 3]
    _decode(b, st, q, sinks, lists, rows, queued, block, delay)
    if queued:
        assert float(st.scores.abs().sum()) == 0.0  # queued until flushed
        for r, sl in zip(rows, lists):
            st.req_to_token[r, :sl.numel()] = sl.int()
        ge.flush(st)
    want = _oracle_counters(b, q, sinks, lists, [np.arange(n) for n in lengths], [n - 1 for n in lengths], block,
                            delay)
    expected = torch.zeros_like(st.scores)
    expected[0] = torch.tensor(want, dtype=torch.float32)
    torch.testing.assert_close(st.scores, expected, rtol=2e-3, atol=1e-6)
    credited = sum(max(0, (n - delay) // block) for n in lengths)
    assert int((st.scores[0, 0] != 0).sum()) == credited


def test_queued_block_counters_over_steps_equal_eager():
    """Five steps with growing lists: the queue's step-by-step counters equal the eager ones."""
    results = {}
    for queued in (False, True):
        ge.STATE = None
        b = backend(gen=torch.Generator().manual_seed(1))
        st = ge.state(b)
        perm = (torch.randperm(19999, generator=torch.Generator().manual_seed(2))[:3000] + 1).cuda()
        sinks = torch.randn(64, generator=torch.Generator().manual_seed(5)).cuda()
        base = [130, 1401]
        for t in range(5):
            q = torch.randn((2, 64, 64), generator=torch.Generator().manual_seed(10 + t)).to(torch.bfloat16).cuda()
            lists = [perm[:base[0] + t], perm[1500:1500 + base[1] + t]]
            _decode(b, st, q, sinks, lists, [1, 2], queued, 4, 3)
        st.req_to_token[1, :base[0] + 4] = perm[:base[0] + 4].int()
        st.req_to_token[2, :base[1] + 4] = perm[1500:1500 + base[1] + 4].int()
        ge.flush(st)
        results[queued] = st.scores.clone()
    torch.testing.assert_close(results[True], results[False], rtol=1e-5, atol=1e-8)
    assert float(results[True][:, 1:].abs().sum()) == 0.0  # only KV head 0 holds counters


@pytest.mark.parametrize("queued", [False, True])
@pytest.mark.parametrize("block,delay", [(4, 128), (16, 0)])
def test_block_counters_after_an_eviction_follow_positions(queued, block, delay):
    """A row after a block boundary: its table holds 70 kept whole blocks of [0, 2048) in position
    order, then req_to_token's tail from frontier 2048 to 2500. The kernels block the list by
    index; the oracle blocks it by position."""
    rng = np.random.default_rng(block)
    g = torch.Generator().manual_seed(4)
    b = backend(gen=g, rows=3)
    st = ge.state(b)
    kept = np.sort(rng.choice(2048 // block, size=70 if block == 16 else 300, replace=False))
    kept_pos = (kept[:, None] * block + np.arange(block)).reshape(-1)
    frontier, n = 2048, 2500
    slots = torch.randperm(19999, generator=g)[:kept_pos.size + n - frontier] + 1
    table, tail = slots[:kept_pos.size], slots[kept_pos.size:]
    st.table[1, :table.numel()] = table.int().cuda()
    st.count[1], st.frontier[1] = table.numel(), frontier
    st.req_to_token[1, frontier:n] = tail.int().cuda()
    listed = torch.zeros(table.numel() + tail.numel(), dtype=torch.int32, device="cuda")
    ge.fill(b, 1, torch.tensor([n], device="cuda"), torch.tensor([1], device="cuda"), listed)
    assert torch.equal(listed.cpu(), torch.cat((table, tail)).int())
    q = torch.randn((1, 64, 64), generator=g).to(torch.bfloat16).cuda()
    sinks = torch.randn(64, generator=g).to(torch.bfloat16).cuda()
    _decode(b, st, q, sinks, [listed.long()], [1], queued, block, delay)
    if queued:
        ge.flush(st)
    positions = np.concatenate((kept_pos, np.arange(frontier, n)))
    want = _oracle_counters(b, q, sinks, [listed.long()], [positions], [n - 1], block, delay)
    expected = torch.zeros_like(st.scores)
    expected[0] = torch.tensor(want, dtype=torch.float32)
    torch.testing.assert_close(st.scores, expected, rtol=2e-3, atol=1e-6)


def _prefill_case(count, prefix_len, seed, slots=20000):
    g = torch.Generator().manual_seed(seed)
    b = backend(gen=g, slots=slots)
    st = ge.state(b)
    q = (torch.randn((count, 64, 64), generator=g) * 1.5).to(torch.bfloat16).cuda()
    sinks = torch.randn(64, generator=g).to(torch.bfloat16).cuda()
    perm = torch.randperm(slots - 1, generator=g)[:prefix_len + count] + 1
    return b, st, q, sinks, perm[:prefix_len].cuda(), perm[prefix_len:].cuda()


@pytest.mark.parametrize("count,prefix_len,block,delay", [
    (1, 0, 4, 0), (37, 0, 4, 0), (100, 300, 16, 0), (257, 1000, 4, 128), (130, 64, 64, 100), (20, 32, 2, 5),
    (16, 4000, 1, 0), (300, 0, 8, 299)])
def test_prefill_block_counters_match_the_oracle(count, prefix_len, block, delay):
    b, st, q, sinks, prefix, new = _prefill_case(count, prefix_len, seed=count + prefix_len + block)
    keys = b.token_to_kv_pool.get_key_buffer(1)
    before = torch.rand(st.scores.shape, generator=torch.Generator().manual_seed(3)).cuda()
    st.scores.copy_(before)
    ge._prefill_scores(st, 0, word(block, delay), layer(1), q, keys, sinks, prefix, new)
    credit, slots = O.prefill_block_step_update(_numpy(q), _numpy(keys), _numpy(sinks), 0.125, 8,
                                                prefix.cpu().numpy(), new.cpu().numpy(), block, delay=delay)
    expected = before.clone()
    expected[0, 0, torch.tensor(slots).cuda()] += torch.tensor(credit, dtype=torch.float32).cuda()
    torch.testing.assert_close(st.scores, expected, rtol=1e-3, atol=1e-6)


def test_prefill_block_counters_over_a_prefix_of_kept_blocks():
    """The prefix is what a block boundary leaves: 120 kept blocks of 4 out of [0, 1000) in
    position order, then the protected recent positions 1000..1199 (more than the delay, so the
    delay never reaches past them); the chunk of 200 queries follows. The oracle blocks by
    position."""
    rng = np.random.default_rng(7)
    kept = np.concatenate((np.sort(rng.choice(250, size=120, replace=False)), np.arange(250, 300)))
    prefix_pos = (kept[:, None] * 4 + np.arange(4)).reshape(-1)
    b, st, q, sinks, prefix, new = _prefill_case(200, prefix_pos.size, seed=77)
    keys = b.token_to_kv_pool.get_key_buffer(1)
    ge._prefill_scores(st, 0, word(4, 128), layer(1), q, keys, sinks, prefix, new)
    credit, slots = O.prefill_block_step_update(_numpy(q), _numpy(keys), _numpy(sinks), 0.125, 8,
                                                prefix.cpu().numpy(), new.cpu().numpy(), 4, prefix_pos, 128)
    expected = torch.zeros_like(st.scores)
    expected[0, 0, torch.tensor(slots).cuda()] = torch.tensor(credit, dtype=torch.float32).cuda()
    torch.testing.assert_close(st.scores, expected, rtol=1e-3, atol=1e-6)
