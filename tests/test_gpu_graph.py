"""Decode steps under HIP graph capture, as SGLang runs them: `fill` and the fused decode of both
full layers (the new tokens' scores zeroed at the first) are captured once and replayed three
times, with eager work and synchronisations between the replays. Every replay's attention output
equals an eager step's bit for bit, and the three replays leave the scores of three eager steps
(queued scores after a flush, or eager scores)."""
from types import SimpleNamespace

import pytest
import torch

from fakes import FULL, backend, layer

pytestmark = pytest.mark.gpu

LENGTHS = [1500, 37, 3001]
ROWS = [1, 2, 3]


@pytest.fixture(autouse=True)
def runtime():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    import gstar_evict
    gstar_evict.STATE = None
    yield gstar_evict
    gstar_evict.STATE = None


def _setup(ge, score_mode):
    g = torch.Generator().manual_seed(41)
    b = backend(gen=g, rows=4, slots=20000)
    st = ge.state(b)
    st.score_mode = score_mode
    perm = torch.randperm(19999, generator=g) + 1
    start = 0
    for r, n in zip(ROWS, LENGTHS):
        st.req_to_token[r, :n] = perm[start:start + n].int().cuda()
        start += n
    st.mode[1], st.mode[2], st.mode[3] = 1, 2, 1
    x = SimpleNamespace(
        b=b, st=st,
        q={lid: torch.randn((3, 64, 64), generator=g).to(torch.bfloat16).cuda() for lid in FULL},
        o={lid: torch.zeros((3, 64, 64), dtype=torch.bfloat16, device="cuda") for lid in FULL},
        sinks=torch.randn(64, generator=g).to(torch.bfloat16).cuda(),
        seq_lens=torch.tensor(LENGTHS, device="cuda"), rows=torch.tensor(ROWS, device="cuda"),
        kv_indices=torch.zeros(sum(LENGTHS), dtype=torch.int32, device="cuda"))
    # The new tokens' slots (zeroed at the first full layer): each row's last list entry.
    x.fb = SimpleNamespace(out_cache_loc=torch.tensor([int(st.req_to_token[r, n - 1]) for r, n in zip(ROWS, LENGTHS)],
                                                      device="cuda"),
                           req_pool_indices=x.rows, seq_lens_cpu=torch.tensor(LENGTHS))
    return x


def _step(ge, x):
    ge.fill(x.b, 3, x.seq_lens, x.rows, x.kv_indices)
    x.b.forward_metadata = SimpleNamespace(kv_indptr=x.b.kv_indptr[:4], kv_indices=x.kv_indices)
    for lid in FULL:
        assert ge.decode(x.b, x.q[lid].view(3, -1), layer(lid), x.fb, x.sinks, x.o[lid].view(3, -1))


@pytest.mark.parametrize("score_mode", ["queue", "eager"])
def test_decode_step_replays_from_a_hip_graph(runtime, score_mode):
    ge = runtime
    # Eager reference: three identical steps (the queue holds all three), then a flush.
    ref = _setup(ge, score_mode)
    outs = []
    for _ in range(3):
        _step(ge, ref)
        outs.append({lid: ref.o[lid].clone() for lid in FULL})
    ge.flush(ref.st)
    torch.cuda.synchronize()
    for step in outs[1:]:
        assert all(torch.equal(step[lid], outs[0][lid]) for lid in FULL)
    want_scores = ref.st.scores.clone()
    assert float(want_scores.abs().sum()) > 0

    ge.STATE = None
    x = _setup(ge, score_mode)
    _step(ge, x)  # warm-up: workspaces and queues exist before capture
    torch.cuda.synchronize()
    x.st.qcount.zero_()
    x.st.scores.zero_()
    for lid in FULL:
        x.o[lid].zero_()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _step(ge, x)
    noise = torch.randn((512, 512), device="cuda")
    for replay in range(3):
        for lid in FULL:
            x.o[lid].zero_()
        graph.replay()
        torch.cuda.synchronize()
        for lid in FULL:
            assert torch.equal(x.o[lid], outs[0][lid]), (replay, lid)
        noise = noise @ noise.t() / 512  # eager work between replays
        torch.cuda.synchronize()
    if score_mode == "queue":
        assert x.st.qcount[:, 1:4].tolist() == [[3, 3, 3]] * len(FULL)
        x.st.queued.update({r: 3 for r in ROWS})
    ge.flush(x.st)
    torch.cuda.synchronize()
    torch.testing.assert_close(x.st.scores, want_scores, rtol=1e-6, atol=1e-9)
