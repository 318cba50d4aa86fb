"""Static regret diagnostic on the GPU (R:549-615) against the oracle, itself pinned to the
reference observer (C:121-232): the reference test T:191-220 at gpt-oss shape (64 query heads,
8 KV heads, d=64), two full layers, a 2200-token prompt in chunks of 2048 and 152."""
from types import SimpleNamespace

import numpy as np
import pytest
import torch

import oracle as O
from fakes import FULL, backend, layer

pytestmark = pytest.mark.gpu

# Each spec takes its own protection (T:240-244): random_2048 protects 64 prefix and 16 recent
# positions, the others 16 and 64 (prefix_sliding: 16 and 884).
SPECS = {"head_sum_2048": (900, 16, 64), "head_max_sum_2048": (900, 16, 64),
         "prefix_sliding_2048": (900, 16, 884), "random_reservoir_2048": (900, 16, 64),
         "random_2048": (900, 64, 16)}


def _random_draws(seed, n, layers, kv_heads, held):
    """random_2048's draws of a diagnostic spec at boundary n: torch's device generator seeded
    with R:573-575's (seed * 1000003 + n * 31 + j) & 0x7FFFFFFF, j the spec's index."""
    j = list(SPECS).index("random_2048")
    generator = torch.Generator(device="cuda")
    generator.manual_seed((seed * 1000003 + n * 31 + j) & 0x7FFFFFFF)
    draws = torch.rand((layers, kv_heads, held), generator=generator, device="cuda", dtype=torch.float64)
    return {j: draws.cpu().numpy()}


@pytest.fixture(autouse=True)
def runtime():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    import gstar_evict
    gstar_evict.STATE = None
    yield gstar_evict
    gstar_evict.STATE = None


def test_lost_mass_and_score_tables_match_the_oracle(runtime):
    ge = runtime
    length = 2200
    g = torch.Generator().manual_seed(17)
    b = backend(rows=2, width=64, slots=length + 8, gen=g)
    st = ge.state(b)
    heads, kv_heads = 64, 8
    queries = {lid: (torch.randn((length, heads, 64), generator=g) * 1.5).to(torch.bfloat16).cuda() for lid in FULL}
    sinks = {lid: torch.randn(heads, generator=g).cuda() for lid in FULL}
    cfg = {"seed": 5, "policies": ",".join(f"{k}:{bb}:{p}:{r}" for k, (bb, p, r) in SPECS.items())}
    req = SimpleNamespace(rid="d", session=None, origin_input_ids=[0] * length)
    e = ge._diagnostic_entry(req, cfg, "cuda", len(FULL), kv_heads)
    oe = O.diagnostic_entry(cfg, length, len(FULL), kv_heads)
    keys_np = {lid: b.token_to_kv_pool.get_key_buffer(lid)[1:length + 1].float().cpu().numpy() for lid in FULL}
    for lo, hi in ((0, 2048), (2048, length)):
        if lo:
            # The boundary at 2048 ranks the GPU's own score tables in both, so residency is exact.
            oe["score_sum"][:] = e["score_sum"].double().cpu().numpy()
            oe["score_max"][:] = e["score_max"].double().cpu().numpy()
        slots = torch.arange(1, hi + 1, device="cuda")
        for index, lid in enumerate(FULL):
            ge._diagnose(st, e, index, layer(lid), queries[lid][lo:hi], b.token_to_kv_pool.get_key_buffer(lid),
                         sinks[lid], slots, lo)
            O.diagnose(oe, index, len(FULL), queries[lid][lo:hi].float().cpu().numpy(), keys_np[lid],
                       sinks[lid].cpu().numpy(), 0.125, kv_heads, lo,
                       random_scores=_random_draws(5, lo, len(FULL), kv_heads, lo) if lo else None)
        torch.cuda.synchronize()
        assert e["error"] is None
        assert np.array_equal(e["resident"].cpu().numpy(), oe["resident"]), (lo, hi)
        np.testing.assert_allclose(e["score_sum"].cpu().numpy(), oe["score_sum"], rtol=2e-3, atol=1e-6)
        np.testing.assert_allclose(e["score_max"].cpu().numpy(), oe["score_max"], rtol=2e-3, atol=1e-6)
    lost = e["lost"].cpu().numpy()
    for j, name in enumerate(SPECS):
        assert oe["lost"][j, 2048:].sum() > 0, name
        np.testing.assert_allclose(lost[j], oe["lost"][j], rtol=1e-3, atol=1e-5, err_msg=name)
    assert e["layers_seen"] == set(FULL)


def test_chunk_across_a_boundary_is_an_error(runtime):
    ge = runtime
    b = backend(rows=2, width=64, slots=4200, gen=torch.Generator().manual_seed(1))
    st = ge.state(b)
    req = SimpleNamespace(rid="d", session=None, origin_input_ids=[0] * 4100)
    e = ge._diagnostic_entry(req, {"seed": 0, "policies": "head_sum_2048:900:16:64"}, "cuda", len(FULL), 8)
    q = torch.zeros((100, 64, 64), dtype=torch.bfloat16, device="cuda")
    ge._diagnose(st, e, 0, layer(FULL[0]), q, b.token_to_kv_pool.get_key_buffer(FULL[0]), torch.zeros(64, device="cuda"),
                 torch.arange(1, 2100, device="cuda"), 2000)
    assert "crosses a boundary" in e["error"]


def test_hooks_write_the_diagnostic_payload(runtime, tmp_path, monkeypatch):
    """`gstar_diagnostic` through the hooks: on_extend creates the entry, after_extend scores each
    chunk per full layer, release writes {"kind": "diagnostic", specs, layers, lost} (R:728-731)."""
    import sys
    import types
    from gstar_evict import retention
    ge = runtime
    monkeypatch.setenv("GSTAR_PAYLOAD_DIR", str(tmp_path))
    names = ["sglang", "sglang.srt", "sglang.srt.mem_cache", "sglang.srt.mem_cache.unified_cache",
             "sglang.srt.mem_cache.unified_cache.component_type"]
    for name in names:
        monkeypatch.setitem(sys.modules, name, types.ModuleType(name))
    sys.modules[names[-1]].ComponentType = SimpleNamespace(SWA="swa")
    length, row = 2100, 1
    g = torch.Generator().manual_seed(3)
    b = backend(rows=2, width=length + 8, slots=length + 8, gen=g)
    st = ge.state(b)
    cfg = {"seed": 2, "policies": "head_sum_2048:1000:16:64,random_reservoir_2048:1000:16:64"}
    req = SimpleNamespace(rid="diag1", session=None, retraction_count=0, origin_input_ids=[0] * length,
                          sampling_params=SimpleNamespace(custom_params={"gstar_diagnostic": cfg}),
                          kv=SimpleNamespace(req_pool_idx=row, holds_kv=True, get_evicted_seqlen=lambda kind: 0))
    batch = SimpleNamespace(reqs=[req], tree_cache=SimpleNamespace(token_to_kv_pool_allocator=None))
    slot_of = torch.arange(1, length + 1, device="cuda")
    st.req_to_token[row, :length] = slot_of.int()
    rows = torch.tensor([row], device="cuda")
    for lo, hi in ((0, 2048), (2048, length)):
        req.extend_range = SimpleNamespace(start=lo, length=hi - lo)
        ge.on_extend(batch)
        b.forward_metadata = SimpleNamespace(qo_indptr=torch.tensor([0, hi - lo], device="cuda"),
                                             kv_indptr=torch.tensor([0, lo], device="cuda", dtype=torch.int32),
                                             kv_indices=slot_of[:lo].int())
        fb = SimpleNamespace(req_pool_indices=rows, out_cache_loc=slot_of[lo:hi], extend_prefix_lens_cpu=[lo])
        for lid in FULL:
            q = torch.randn((hi - lo, 64, 64), generator=g).to(torch.bfloat16).cuda()
            ge.after_extend(b, q.reshape(hi - lo, -1), layer(lid), fb, torch.zeros(64, device="cuda"))
    entry = st.entries[row]
    assert entry["kind"] == "diagnostic" and entry["error"] is None
    ge.release(req)
    payload = retention.read_payload(tmp_path / "diag1.json.gz")
    assert payload["kind"] == "diagnostic" and payload["layers"] == list(FULL)
    assert [tuple(s) for s in payload["specs"]] == [("head_sum_2048", 1000, 16, 64),
                                                    ("random_reservoir_2048", 1000, 16, 64)]
    assert payload["lost"].shape == (2, length)
    assert np.array_equal(payload["lost"], entry["lost"].cpu().numpy())
    assert payload["lost"][:, :2048].sum() == 0 and payload["lost"][:, 2048:].min() > 0
    assert row not in st.entries
