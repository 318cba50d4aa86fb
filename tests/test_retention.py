"""Retention records (R:500-507) and their reader (sglang_client.py:115-133 behaviour).

The writer's format is the runtime's own `array` / `write_payload`; victims come from
`core.Policy`'s per-head resident sets (C:33-118) over several boundaries, and the rebuilt
retained sets must equal those resident sets after every boundary. The GPU test of the
product's `_boundary` writer is in test_gpu_boundary.py.
"""
import numpy as np
import pytest

import oracle as O


@pytest.fixture
def runtime(tmp_path, monkeypatch):
    monkeypatch.setenv("GSTAR_PAYLOAD_DIR", str(tmp_path))
    import gstar_evict
    from gstar_evict import retention
    return gstar_evict, retention, tmp_path


def test_array_envelope_round_trip(runtime):
    ge, R, _ = runtime
    for dtype, values in (("uint32", [0, 5, 2 ** 32 - 1]), ("int32", [[1, -2], [3, 4]]), ("float64", [0.5, -1e300])):
        got = R.decode_array(ge.array(values, dtype))
        assert got.dtype == np.dtype(dtype) and np.array_equal(got, np.asarray(values, dtype=dtype))


def test_retained_sets_rebuild_policy_resident_sets(runtime):
    ge, R, tmp = runtime
    layers, heads, budget, prefix, recent = 2, 3, 300, 20, 40
    rng = np.random.default_rng(5)
    policies = [O.Policy("head_sum_2048", budget, prefix, recent, seed=1, stream=(l, g))
                for l in range(layers) for g in range(heads)]
    held_before = [set() for _ in policies]
    expected = {}
    for n in (512, 1024, 1536, 2048):
        victims = []
        for i, p in enumerate(policies):
            for t in range(p.next_position, n):
                p.append(t)
            p.scores = {t: float(rng.random()) for t in p.resident}
            before = held_before[i] | set(range(n - 512, n))
            p.finish()
            victims.append(np.array(sorted(before - p.resident), dtype=np.int64))
            held_before[i] = set(p.resident)
        deltas = np.concatenate([np.diff(v, prepend=0) for v in victims])
        ge.write_payload(f"r-b{n}", {"kind": "retention", "boundary": n, "cfg": {}, "layers": list(range(layers)),
                                     "kv_heads": heads, "evicted_delta": ge.array(deltas, "uint32"),
                                     "evicted_counts": ge.array([len(v) for v in victims], "int32")})
        expected[n] = [sorted(p.resident) for p in policies]
    records = [R.read_payload(path) for path in sorted(tmp.glob("r-b*.json.gz"))]
    assert all(r["format"] == "gstar-payload-1" for r in records)
    seen = []
    for n, held in R.retained_sets(records):
        seen.append(n)
        assert [h.tolist() for h in held] == expected[n], n
    assert seen == [512, 1024, 1536, 2048]


def test_counts_must_cover_deltas(runtime):
    _, R, _ = runtime
    with pytest.raises(ValueError):
        R.evicted_per_head({"evicted_counts": np.array([2, 2]), "evicted_delta": np.array([1, 2, 3])})
