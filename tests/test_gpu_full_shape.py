"""The bs=32 decode workload at full size, checked through properties that do not depend on size:
12 full-attention layers of gpt-oss-20b shape, 32 sequences of 16K-64K tokens (random 16-token
pages), a 32,768-position budget (512 + 4096 + 28,160), head_sum, a boundary every 64 decode
steps (bench.py's default workload, built by its own Workload class).

At the first evicting boundary the test takes the row's flushed scores and K/V, lets the decode
hook's path run the boundary (queued, finished at the next step), and checks that every (layer,
KV head) keeps exactly the positions the oracle's `choose` keeps on the same scores (bit-exact),
that the new table's slots hold, for every head, the K, V and score of the position the head
claims (first and last layer), and that the row owns each table slot once.
"""
import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu


def test_boundary_at_the_bs32_32k_budget_decode_shape():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    import bench
    import gstar_evict as ge
    args = bench.parse(["--steps", "80", "--warmup", "0", "--no-cpu-baseline"])
    w = bench.Workload(args, torch, ge)
    st, pool = w.st, w.backend.token_to_kv_pool
    for _ in range(70):
        due = [i for i, e in enumerate(w.entries)
               if w.lens[i] % args.interval == 0 and w.lens[i] > e["last_boundary"] and e["count"]]
        if due:
            break
        w.step(account=False)
    assert due, "no boundary within 70 steps"
    i = due[0]
    row, e, n = i + 1, w.entries[i], w.lens[i]
    ge.flush(st, [row])  # the boundary's own flush then finds an empty queue
    c, f = e["count"], e["frontier"]
    slots = torch.cat((st.table[row, :c], st.req_to_token[row, f:n])).long()
    N = slots.numel()
    pos = torch.empty((args.layers, 8, N), dtype=torch.int64, device="cuda")
    pos[..., :c] = e["pos"].long()
    pos[..., c:] = torch.arange(f, n, device="cuda")
    scores = st.scores[:, :, slots].clone()
    checked = (0, args.layers - 1)
    k_before = {l: pool.get_key_buffer(l)[slots].clone() for l in checked}
    v_before = {l: pool.get_value_buffer(l)[slots].clone() for l in checked}

    w.step(account=False)  # queues the boundary (and any others due), then decodes
    ge.finish_boundaries(st)
    torch.cuda.synchronize()
    assert e["count"] == args.budget and e["frontier"] == n

    # Selection: the oracle's choose on the same float32 scores (compared as float64).
    keep, protected = O.choose("head_sum_2048", pos.cpu().numpy(), n, args.budget, args.prefix, args.recent,
                               scores.double().cpu().numpy(), n - 256)
    want = np.take_along_axis(pos.cpu().numpy(), keep, -1)
    got = e["pos"].long().cpu().numpy()
    assert protected == args.prefix + args.recent
    assert np.array_equal(np.sort(got, -1), np.sort(want, -1))

    # Relocation: the table's slots hold each head's claimed positions' K, V and score.
    table = st.table[row, :e["count"]].long()
    heads = torch.arange(8, device="cuda")[:, None]
    for l in checked:
        column_of = torch.full((8, n), -1, dtype=torch.int64, device="cuda")
        column_of.scatter_(1, pos[l], torch.arange(N, device="cuda").expand(8, -1).contiguous())
        cols = column_of.gather(1, e["pos"][l].long())  # [8, count]: the pre-boundary column of each claim
        assert bool((cols >= 0).all())
        assert torch.equal(pool.get_key_buffer(l)[table].transpose(0, 1), k_before[l][cols, heads])
        assert torch.equal(pool.get_value_buffer(l)[table].transpose(0, 1), v_before[l][cols, heads])
        assert torch.equal(st.scores[l][:, table], scores[l].gather(1, cols))
    assert table.unique().numel() == table.numel()
