"""Reading the runtime's payloads and rebuilding retained sets from retention records.

A payload is a gzip'd JSON object (`format` "gstar-payload-1", R:71-76) whose numpy arrays
travel as `{"dtype", "shape", "data"}` with base64 data (R:66-68). A retention record, written
by `_boundary` for configs with `record` (R:500-507), holds for one boundary at logical length
`boundary` the evicted positions of every (full layer, KV head), layer-major: ascending and
delta-coded within each head (`evicted_delta`, uint32) with one count per head
(`evicted_counts`, int32).

`retained_sets` replays records into the positions each head holds after every boundary, the
client-side reading of the same records (sglang_client.py:115-133): before a boundary a head
holds its previous survivors plus every position since the previous record (boundaries that
evict nothing write no record), and the boundary removes its victims.
"""
from __future__ import annotations

import numpy as np

from .payloads import decode_array, decode_arrays, read as read_payload  # noqa: F401  (reader API)


def evicted_per_head(record):
    """The record's evicted positions, one ascending int64 array per layer-major (layer, head)."""
    counts = np.asarray(record["evicted_counts"], dtype=np.int64)
    deltas = np.asarray(record["evicted_delta"], dtype=np.int64)
    if counts.sum() != deltas.size:
        raise ValueError("retention record: counts do not cover the deltas")
    ends = np.cumsum(counts)
    return [np.cumsum(deltas[end - c:end]) for c, end in zip(counts, ends)]


def retained_sets(records):
    """Yield (boundary, held) after every record, held[i] = sorted positions of head i."""
    held, last = None, 0
    for record in sorted(records, key=lambda r: r["boundary"]):
        n = int(record["boundary"])
        victims = evicted_per_head(record)
        arriving = np.arange(last, n, dtype=np.int64)
        if held is None:
            held = [arriving] * len(victims)
        elif len(held) != len(victims):
            raise ValueError("retention records disagree on the number of heads")
        else:
            held = [np.concatenate((h, arriving)) for h in held]
        held = [h[~np.isin(h, v)] for h, v in zip(held, victims)]
        last = n
        yield n, held
