"""Fake SGLang objects for driving the runtime hooks, after the reference test's fakes (T:19-39)."""
from types import SimpleNamespace

import torch

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
