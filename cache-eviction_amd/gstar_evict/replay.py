"""Static replay's layer difference (``_replay_layer_difference``, R:520-546).

A replay entry keeps the first full layer's unevicted keys and values by position (the
shadow). For every prefill chunk, that layer's attention output over all of them (a) is
compared with the output over each KV head's survivors (b): the retained positions, then
everything from the frontier on. The layer before it is a sliding-window layer, so its input
does not depend on eviction and the difference isolates this layer's loss. One
``gse_replay_layer_difference`` call computes both outputs (MFMA, single-pass online softmax)
and the per-query ``|b - a| / max(|a|, 1e-12)``.
"""
from __future__ import annotations

import numpy as np
import torch

from . import _native as N


def _retained(entry):
    """Each KV head's retained positions of the first full layer as int32 [G, count] with unit
    column stride, or None before the first eviction."""
    if not entry["count"]:
        return None
    pos = entry["pos"][0]
    if pos.dtype != torch.int32 or pos.stride(1) != 1:
        pos = pos.to(torch.int32).contiguous()
    return pos


def layer_difference(st, entry, queries, layer, sinks, start):
    """Queue one chunk's errors (queries ``[count, heads, dim]`` at positions ``start``..) and
    keep them, on the device, in ``entry["layer_error"]``."""
    count = queries.shape[0]
    heads, kv_heads = layer.tp_q_head_num, layer.tp_k_head_num
    sk, sv = entry["shadow_k"], entry["shadow_v"]
    retained = _retained(entry)
    error = torch.empty(count, dtype=torch.float32, device=queries.device)
    ws = st.workspace("replay", N.lib().gse_replay_workspace_bytes(count, heads))
    N.call("gse_replay_layer_difference", N.ptr(queries), queries.stride(0), queries.stride(1), count, N.ptr(sk),
           N.ptr(sv), sk.stride(0), sk.stride(1), sk.shape[0], start, N.ptr(retained),
           retained.stride(0) if retained is not None else 0, retained.shape[1] if retained is not None else 0,
           entry["frontier"], N.ptr(sinks), N.float_code(sinks), heads, kv_heads, layer.qk_head_dim,
           float(layer.scaling), N.ptr(error), N.ptr(ws), ws.numel(), N.stream())
    entry["layer_error"].append(error)


def collected(entry):
    """Every chunk's errors in query order, float32 on the host."""
    if not entry["layer_error"]:
        return np.zeros(0, dtype=np.float32)
    return torch.cat(entry["layer_error"]).cpu().numpy()
