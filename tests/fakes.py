"""Fake SGLang objects for driving the runtime hooks, after the reference test's fakes (T:19-39),
and the oracle-side mirror of a fake backend's state."""
from types import SimpleNamespace

import numpy as np
import torch

import oracle as O

FULL = (1, 3)


def backend(rows=4, width=8192, slots=20000, splits=8, kv_heads=8, dim=64, layers=4, full=FULL, gen=None,
            device="cuda"):
    """Full layers `full`, the others sliding-window; distinct random bf16 keys and values per layer."""
    def rnd():
        return torch.randn((slots, kv_heads, dim), generator=gen).to(torch.bfloat16).to(device)

    keys = {l: rnd() for l in range(layers)}
    values = {l: rnd() for l in range(layers)}
    pool = SimpleNamespace(layers_mapping={l: (l, l not in full) for l in range(layers)},
                           get_key_buffer=keys.__getitem__, get_value_buffer=values.__getitem__)
    return SimpleNamespace(token_to_kv_pool=pool, max_kv_splits=splits,
                           req_to_token_pool=SimpleNamespace(req_to_token=torch.zeros(
                               (rows, width), dtype=torch.int32, device=device)),
                           kv_indptr=torch.zeros(rows + 1, dtype=torch.int32, device=device))


def allocator(slots=20000, device="cuda"):
    freed = []
    return freed, SimpleNamespace(free_full=lambda s: freed.append(s.clone()),
                                  full_to_swa_index_mapping=torch.zeros(slots, dtype=torch.int64, device=device))


def entry(ge, name, budget, prefix, recent, seed, kind="live", record=False):
    cfg = {"name": name, "budget": budget, "prefix": prefix, "recent": recent, "seed": seed, "record": record}
    return ge._live_entry(SimpleNamespace(rid="r", session=None), cfg, kind)


def layer(layer_id, heads=64, kv_heads=8, dim=64, scaling=0.125):
    return SimpleNamespace(sliding_window_size=-1, tp_q_head_num=heads, tp_k_head_num=kv_heads,
                           qk_head_dim=dim, layer_id=layer_id, scaling=scaling)


def oracle_state(b, st, full=FULL):
    """The oracle's copy of the backend's full-layer pools, req_to_token and scores."""
    keys = [b.token_to_kv_pool.get_key_buffer(l).float().cpu().numpy() for l in full]
    values = [b.token_to_kv_pool.get_value_buffer(l).float().cpu().numpy() for l in full]
    return O.OracleState(keys, values, st.req_to_token.cpu().numpy(), st.scores.cpu().numpy())


def assert_same_state(b, st, ost, e, oe, row, n_rows, full=FULL):
    """After the same boundary on the GPU and in the oracle: entries, table, counts, retained
    positions, req_to_token of the first n_rows rows, scores and pools are identical."""
    assert e["count"] == oe["count"] and e["frontier"] == oe["frontier"]
    assert np.array_equal(st.table[row, :e["count"]].cpu().numpy(), ost.table[row, :oe["count"]])
    assert int(st.count[row]) == e["count"] and int(st.frontier[row]) == e["frontier"]
    assert np.array_equal(e["pos"].cpu().numpy(), oe["pos"])
    assert np.array_equal(st.req_to_token[:n_rows].cpu().numpy(), ost.req_to_token[:n_rows])
    assert np.array_equal(st.scores.cpu().numpy(), ost.scores)
    for index, l in enumerate(full):
        assert np.array_equal(b.token_to_kv_pool.get_key_buffer(l).float().cpu().numpy(), ost.keys[index])
        assert np.array_equal(b.token_to_kv_pool.get_value_buffer(l).float().cpu().numpy(), ost.values[index])
