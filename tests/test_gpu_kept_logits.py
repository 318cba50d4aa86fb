"""Kept decode products: rows whose boundary is due at the next step keep the step's q.k products
(fp32, written by the fused decode kernel), and the flush folds such a one-step queue from them
with gse_score_flush_logits instead of reading K again. Its scores equal the short-queue flush's
bit for bit, so whole eviction flows are identical with and without it."""
from types import SimpleNamespace

import pytest
import torch

from fakes import FULL, backend, layer

pytestmark = pytest.mark.gpu


@pytest.fixture()
def ge():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    import gstar_evict
    gstar_evict.STATE = None
    yield gstar_evict
    gstar_evict.STATE = None


def _calls(monkeypatch):
    """Record the entry points the runtime calls."""
    from gstar_evict import _native as N
    names = []
    real = N.call

    def spy(name, *args):
        names.append(name)
        return real(name, *args)

    monkeypatch.setattr(N, "call", spy)
    return names


def _run(ge, kv_heads, delay, keep):
    """Two decode steps of rows 1 (sum), 2 (max) and 3 (sum); rows 1 and 2 are flushed after the
    first, so at the second only their queues hold one step: with ``keep`` they keep its products.
    Returns the scores after a flush of every row, and the second step's products and inputs."""
    from gstar_evict import attention
    heads = 8 * kv_heads
    b = backend(gen=torch.Generator().manual_seed(1), kv_heads=kv_heads)
    st = ge.state(b)
    st.score_mode = "queue"
    for r, kind in ((1, 1), (2, 2), (3, 1)):
        st.mode[r] = kind | delay << 8
        st.entries[r] = {"mode": kind}
    base = [100, 1301, 2000]
    perm = (torch.randperm(19999, generator=torch.Generator().manual_seed(2))[:6000] + 1).cuda()
    starts = [0, 1500, 3000]
    sinks = torch.randn(heads, generator=torch.Generator().manual_seed(5)).cuda()
    rows = [1, 2, 3]
    for r, s0, n in zip(rows, starts, base):
        st.req_to_token[r, :n + 2] = perm[s0:s0 + n + 2].int()
    kept = None
    for t in range(2):
        attention.begin_decode_step(st, rows, rows if (keep and t == 1) else ())
        lens = [n + t for n in base]
        idx = torch.cat([perm[s0:s0 + n] for s0, n in zip(starts, lens)])
        indptr = torch.tensor([0, lens[0], lens[0] + lens[1], sum(lens)], dtype=torch.int32, device="cuda")
        b.forward_metadata = SimpleNamespace(kv_indptr=indptr, kv_indices=idx)
        fb = SimpleNamespace(out_cache_loc=idx[indptr[1:].long() - 1], req_pool_indices=torch.tensor(rows, device="cuda"),
                             seq_lens_cpu=torch.tensor(lens))
        q = torch.randn((3, heads, 64), generator=torch.Generator().manual_seed(10 + t)).to(torch.bfloat16).cuda()
        o = torch.empty((3, heads, 64), dtype=torch.bfloat16, device="cuda")
        for lid in FULL:
            ge.decode(b, q.reshape(3, -1), layer(lid, heads=heads, kv_heads=kv_heads), fb, sinks, o.reshape(3, -1))
        if t == 0:
            ge.flush(st, [1, 2])
        elif keep:
            lrows, lcap = st.logit_layout
            buf = st.workspace("logits", 0)[:4 * lrows * lcap * heads * len(FULL)].view(torch.float32)
            planes = buf.view(len(FULL), lrows, kv_heads, lcap, 8)  # a plane of 8 heads per KV head
            kept = (planes.permute(0, 1, 3, 2, 4).reshape(len(FULL), lrows, lcap, heads).clone(),
                    dict(st.logit_rows_on_device), q, idx, lens, b)
    ge.flush(st)
    torch.cuda.synchronize()
    return st.scores.clone(), kept


@pytest.mark.parametrize("kv_heads,delay", [(8, 0), (8, 7), (4, 0)])
def test_logit_flush_equals_the_short_flush_bit_for_bit(ge, monkeypatch, kv_heads, delay):
    plain = _run(ge, kv_heads, delay, keep=False)[0]
    ge.STATE = None
    names = _calls(monkeypatch)
    scores, (logits, index, q, idx, lens, b) = _run(ge, kv_heads, delay, keep=True)
    assert names.count("gse_score_flush_logits") == 1  # rows 1 and 2 in one launch; row 3 folds two steps
    assert set(index) == {1, 2}
    assert float(plain.abs().sum()) > 0
    assert torch.equal(scores, plain)
    # The kept products are q.k of each listed key (fp32 accumulation of bf16 products).
    heads = 8 * kv_heads
    group = heads // kv_heads
    for i, r in enumerate((1, 2)):
        off = sum(lens[:i])
        slots = idx[off:off + lens[i]].long()
        for li, lid in enumerate(FULL):
            keys = b.token_to_kv_pool.get_key_buffer(lid)[slots].float()  # [n, G, D]
            want = torch.einsum("hd,nhd->nh", q[i].float(), keys.repeat_interleave(group, dim=1))
            got = logits[li, index[r], :lens[i]]
            torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-4)


def test_eviction_at_every_step_is_identical_with_kept_products(ge, monkeypatch):
    """bench.py's eviction-at-every-step flow (3 sequences of 6-9K tokens, budget 4096) for six
    steps: scores, tables, req_to_token and the relocated K/V pools match bit for bit whether the
    boundaries' flushes read kept products or K."""
    import bench
    from gstar_evict import attention
    args = bench.parse(["--bs", "3", "--min-len", "6000", "--max-len", "9000", "--budget", "4096", "--prefix", "64",
                        "--recent", "512", "--interval", "1", "--layers", "3", "--heavy", "0", "--dup", "0.1",
                        "--steps", "8", "--warmup", "0", "--no-cpu-baseline"])
    real_keep = attention.keep_logits
    states = {}
    for keep in (False, True):
        ge.STATE = None
        monkeypatch.setattr(attention, "keep_logits", real_keep if keep else (lambda st, rows: real_keep(st, [])))
        names = _calls(monkeypatch)
        torch.manual_seed(0)  # the workload's pools and queries come from the default generators
        w = bench.Workload(args, torch, ge)
        for _ in range(6):
            w.step(account=False)
        ge.finish_boundaries(w.st)
        torch.cuda.synchronize()
        pool = w.backend.token_to_kv_pool
        st = w.st
        states[keep] = dict(scores=st.scores.clone(), table=st.table.clone(), r2t=st.req_to_token.clone(),
                            k=[pool.get_key_buffer(l).clone() for l in st.full_layers],
                            v=[pool.get_value_buffer(l).clone() for l in st.full_layers],
                            freed=[e["events"][-1].get("freed") for e in w.entries])
        flushes = names.count("gse_score_flush_logits")
        assert (flushes >= 5) if keep else (flushes == 0), flushes
        monkeypatch.undo()
    a, b = states[False], states[True]
    assert a["freed"] == b["freed"] and all(f == 1 for f in a["freed"])
    for name in ("scores", "table", "r2t"):
        assert torch.equal(a[name], b[name]), name
    for name in ("k", "v"):
        assert all(torch.equal(x, y) for x, y in zip(a[name], b[name])), name
