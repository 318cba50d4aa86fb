// Fused decode attention + per-KV-head H2O score accumulation (gfx950).
//
// One workgroup = one (sequence, split of `chunk` resident keys); its 8 waves
// are the 8 KV heads, so the workgroup streams whole 1 KiB K rows and 1 KiB V
// rows of the pool (each wave a coalesced 128-byte head row per key).
//
// Per 32-key tile a wave does, with v_mfma_f32_16x16x32_bf16:
//   S^T = K . Qcur^T      [16 keys x 16 heads], 8 live heads  (attention logits)
//   Sp  = Qprev . K^T     [16 heads x 16 keys]                 (pending score logits)
//   O^T += V^T . P^T      [16 dims x 16 heads] x 4 dim blocks  (V transposed through LDS)
// The online softmax keeps (m, l) per head in registers; the sink enters in the
// merge. The score update of the pending query uses its final normaliser,
// known since the previous call, so K is read once per step (GSE_SCORE_LAG).
// GSE_SCORE_EAGER runs the attention pass, the merge, then a score-only pass.
#include <type_traits>

#include "common.hpp"

namespace gse {

constexpr int D = 64;        // head_dim
constexpr int GROUP = 8;     // query heads per KV head
constexpr int TILE = 64;     // keys per inner iteration (four 16-key MFMA sub-tiles)
constexpr int MAX_KVH = 8;   // waves per workgroup
constexpr int LDS_ROW = D + 16;  // padded bf16 row of the V staging tile (160 B: transposed reads spread over banks)
constexpr int PART = D + 4;     // floats per (sequence, split, head) partial: o[64], m, l, pad (16-byte rows)

struct SlotSrc {
  // CSR (fill output): slot(b, i) = indices[indptr[b] + i], length indptr[b+1] - indptr[b].
  const int32_t* indptr;
  const void* indices;
  // Row view (flush): slot(r, i) = i < count[r] ? table[r, i] : req_to_token[r, frontier[r] + i - count[r]].
  const int32_t* table;
  int64_t table_stride;
  const int32_t* r2t;
  int64_t r2t_stride;
  int64_t r2t_width;
  const int32_t* frontier;
  const int32_t* count;
};

struct DecodeArgs {
  const uint16_t* q;
  int64_t q_sb, q_sh;
  const uint16_t* k;
  const uint16_t* v;
  int64_t kv_ss, kv_sh;
  SlotSrc src;
  const void* sinks;
  int sinks_dtype;
  const int32_t* mode;
  const void* rows;
  int rows_dtype;
  float* scores;
  int64_t scores_sg, scores_ss;
  // Score query / normaliser / length source.
  const uint16_t* sq;
  int64_t sq_sb, sq_sh;
  const float* snorm;
  int64_t snorm_sb;
  const int32_t* slen;  // per row (LAG / flush); null -> CSR length (EAGER)
  int score_by_row;     // index sq/snorm by row (1) or by batch entry (0)
  float* part;          // [bs, max_splits, q_heads, PART]
  int q_heads, kv_heads, chunk, max_splits;
  float scale2;         // sm_scale * log2(e)
};

GSE_DEVICE int64_t row_of(const DecodeArgs& a, int b) { return load_index_dyn(a.rows, a.rows_dtype, b); }

template <bool ROWVIEW, typename IdxT>
GSE_DEVICE int64_t fetch_slot(const SlotSrc& s, int64_t row, int64_t base, int64_t cnt, int64_t fr, int64_t i) {
  if constexpr (ROWVIEW) {
    return i < cnt ? int64_t(s.table[row * s.table_stride + i]) : int64_t(s.r2t[row * s.r2t_stride + fr + i - cnt]);
  } else {
    return int64_t(static_cast<const IdxT*>(s.indices)[base + i]);
  }
}

GSE_DEVICE uint4 ld16(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }

// ATTN: attention partials for the current query. SCORE: score update of the
// score query (pending or current). ROWVIEW: slot list from the eviction state.
//
// Software pipeline per 64-key tile t: the slot indices of tile t+2, then the
// K/V rows and old scores of tile t+1 are issued before tile t is computed, so
// no load on the critical path waits for a dependent load.
template <bool ATTN, bool SCORE, bool ROWVIEW, typename IdxT>
__global__ __launch_bounds__(512) void decode_split_kernel(DecodeArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t vtile[MAX_KVH][TILE * LDS_ROW];

  const int b = blockIdx.y;
  const int split = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int g = threadIdx.x >> 6;
  if (g >= a.kv_heads) return;
  const int col = lane & 15;
  const int grp = lane >> 4;

  const int64_t row = row_of(a, b);
  int64_t base = 0, len = 0, cnt = 0, fr = 0;
  if constexpr (ROWVIEW) {
    cnt = a.src.count[row];
    fr = a.src.frontier[row];
  } else {
    base = a.src.indptr[b];
    len = int64_t(a.src.indptr[b + 1]) - base;
  }

  bool do_score = false;
  int64_t slen = 0;
  if constexpr (SCORE) {
    const int md = a.mode[row];
    slen = a.slen ? int64_t(a.slen[row]) : len;
    // A pending list is a prefix of the current one; never read past either list.
    if constexpr (ROWVIEW) {
      const int64_t cap = cnt + a.src.r2t_width - fr;
      slen = slen < cap ? slen : cap;
      len = slen;
    } else {
      slen = slen < len ? slen : len;
    }
    do_score = (md == 1 || md == 2) && slen > 0;
  }
  const int64_t k0 = int64_t(split) * a.chunk;
  const int64_t attn_end = ATTN ? (k0 + a.chunk < len ? k0 + a.chunk : len) : 0;
  const int64_t score_end = do_score ? (k0 + a.chunk < slen ? k0 + a.chunk : slen) : 0;
  const int64_t k_end = attn_end > score_end ? attn_end : score_end;
  if (k0 >= k_end) return;
  const bool max_mode = SCORE ? (a.mode[row] == 2) : false;

  // Query fragments: lane supplies head (g*8 + col) dims [16*grp, 16*grp + 16), zero for col >= 8.
  bf16x8_t qc0 = {}, qc1 = {}, qp0 = {}, qp1 = {};
  const int hq = g * GROUP + col;
  if (col < GROUP) {
    if constexpr (ATTN) {
      const uint16_t* qp = a.q + int64_t(b) * a.q_sb + int64_t(hq) * a.q_sh + 16 * grp;
      qc0 = as_bf16x8(ld16(qp));
      qc1 = as_bf16x8(ld16(qp + 8));
    }
    if (do_score) {
      const int64_t si = a.score_by_row ? row : b;
      const uint16_t* qp = a.sq + si * a.sq_sb + int64_t(hq) * a.sq_sh + 16 * grp;
      qp0 = as_bf16x8(ld16(qp));
      qp1 = as_bf16x8(ld16(qp + 8));
    }
  }
  // Pending normalisers of heads 4*grp + r (rows of Sp); only grp < 2 are live.
  float pn[4] = {0.f, 0.f, 0.f, 0.f};
  if (do_score && grp < 2) {
    const int64_t si = a.score_by_row ? row : b;
#pragma unroll
    for (int r = 0; r < 4; ++r) pn[r] = a.snorm[si * a.snorm_sb + g * GROUP + 4 * grp + r] * kLog2e;
  }

  float m_run = -INFINITY, l_run = 0.f;
  f32x4_t oacc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) oacc[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const uint16_t* kbase = a.k + int64_t(g) * a.kv_sh + 16 * grp;
  const uint16_t* vbase = a.v + int64_t(g) * a.kv_sh + 16 * grp;
  uint16_t* vt = vtile[g];
  float* srow = a.scores + int64_t(g) * a.scores_sg;

  // Slot of key i of this split (slot 0, the null slot, past the end). The index load is
  // issued unconditionally (clamped to the last key) so every path issues the same loads and
  // the compiler's wait counts stay exact.
  auto slot_at = [&](int64_t i) -> int32_t {
    const int32_t s = int32_t(fetch_slot<ROWVIEW, IdxT>(a.src, row, base, cnt, fr, i < k_end ? i : k_end - 1));
    return i < k_end ? s : 0;
  };
  const int ntiles = int((k_end - k0 + TILE - 1) / TILE);
  const bool score_live = SCORE && do_score;

  // One 64-key tile: slots of keys (tb + 16*st + col), K/V 16-dim halves, old score of key tb + lane.
  struct Tile {
    int32_t s[4];
    uint4 k[4][2], v[4][2];
    float osc;
  };
  // Slot of the key this lane owns in the score update (sub-tile grp); no dynamic
  // register indexing, so tiles stay in VGPRs.
  auto own_slot = [&](const Tile& T) -> int32_t {
    return grp == 0 ? T.s[0] : (grp == 1 ? T.s[1] : (grp == 2 ? T.s[2] : T.s[3]));
  };
  auto issue_rows = [&](Tile& T) {
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const uint16_t* kp = kbase + int64_t(T.s[st]) * a.kv_ss;
      T.k[st][0] = ld16(kp);
      T.k[st][1] = ld16(kp + 8);
      if constexpr (ATTN) {
        const uint16_t* vp = vbase + int64_t(T.s[st]) * a.kv_ss;
        T.v[st][0] = ld16(vp);
        T.v[st][1] = ld16(vp + 8);
      }
    }
    if constexpr (SCORE) T.osc = srow[int64_t(score_live ? own_slot(T) : 0) * a.scores_ss];
  };

  // Compute tile t held in X. Lanes of group grp read the V^T fragments of keys
  // 32*half + 16*h + 4*grp + e at dims 16*j + 4*(lane%4) (ds_read_b64_tr_b16).
  auto compute = [&](int t, Tile& X) {
    const int64_t tb = k0 + int64_t(t) * TILE;
    if constexpr (ATTN) {
      if (tb < attn_end) {
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          *reinterpret_cast<uint4*>(vt + (16 * st + col) * LDS_ROW + 16 * grp) = X.v[st][0];
          *reinterpret_cast<uint4*>(vt + (16 * st + col) * LDS_ROW + 16 * grp + 8) = X.v[st][1];
        }
        // S^T sub-tiles: sc[st][r] = q.k (head col, key tb + 16*st + 4*grp + r), unscaled.
        f32x4_t sc[4];
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
          acc = mfma16x16x32(as_bf16x8(X.k[st][0]), qc0, acc);
          sc[st] = mfma16x16x32(as_bf16x8(X.k[st][1]), qc1, acc);
        }
        if (tb + TILE > attn_end) {  // only the last tile of a split is partial
          const int lim = int(attn_end - tb);
#pragma unroll
          for (int st = 0; st < 4; ++st)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (16 * st + 4 * grp + r >= lim) sc[st][r] = -INFINITY;
        }
        float tmax = fmaxf(fmaxf(fmaxf(sc[0][0], sc[0][1]), fmaxf(sc[0][2], sc[0][3])),
                           fmaxf(fmaxf(sc[1][0], sc[1][1]), fmaxf(sc[1][2], sc[1][3])));
        tmax = fmaxf(tmax, fmaxf(fmaxf(fmaxf(sc[2][0], sc[2][1]), fmaxf(sc[2][2], sc[2][3])),
                                 fmaxf(fmaxf(sc[3][0], sc[3][1]), fmaxf(sc[3][2], sc[3][3]))));
        tmax = xor32_max(xor16_max(tmax)) * a.scale2;  // log2 units (scale > 0)
        // Lazy rescale: keep the running maximum unless some head's tile maximum
        // exceeds it by more than 2^8 (exact: O and l share the reference).
        if (__any(tmax > m_run + 8.f)) {
          const float m_new = fmaxf(m_run, tmax);
          const float corr = fast_exp2(m_run - m_new);
          m_run = m_new;
          l_run *= corr;
#pragma unroll
          for (int j = 0; j < 4; ++j) oacc[j] = oacc[j] * corr;
        }
        float psum = 0.f;
#pragma unroll
        for (int st = 0; st < 4; ++st)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            sc[st][r] = fast_exp2(fmaf(sc[st][r], a.scale2, -m_run));
            psum += sc[st][r];
          }
        l_run += psum;
        // P^T operands: half 0 covers sub-tiles 0/1, half 1 sub-tiles 2/3; k-element e maps to
        // sub-tile 2*half + e/4, key 4*grp + e%4.
        uint4 pa, pb;
        pa.x = pack_bf16x2(sc[0][0], sc[0][1]);
        pa.y = pack_bf16x2(sc[0][2], sc[0][3]);
        pa.z = pack_bf16x2(sc[1][0], sc[1][1]);
        pa.w = pack_bf16x2(sc[1][2], sc[1][3]);
        pb.x = pack_bf16x2(sc[2][0], sc[2][1]);
        pb.y = pack_bf16x2(sc[2][2], sc[2][3]);
        pb.z = pack_bf16x2(sc[3][0], sc[3][1]);
        pb.w = pack_bf16x2(sc[3][2], sc[3][3]);
        __builtin_amdgcn_wave_barrier();
        const uint16_t* vr = vt + (4 * grp + ((lane & 15) >> 2)) * LDS_ROW + 4 * (lane & 3);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const s16x4_t a0 = ds_read_tr16(vr + 16 * j);
          const s16x4_t a1 = ds_read_tr16(vr + 16 * LDS_ROW + 16 * j);
          const s16x4_t b0 = ds_read_tr16(vr + 32 * LDS_ROW + 16 * j);
          const s16x4_t b1 = ds_read_tr16(vr + 48 * LDS_ROW + 16 * j);
          oacc[j] = mfma16x16x32(join_bf16x8(a0, a1), as_bf16x8(pa), oacc[j]);
          oacc[j] = mfma16x16x32(join_bf16x8(b0, b1), as_bf16x8(pb), oacc[j]);
        }
        __builtin_amdgcn_wave_barrier();
      }
    }

    if constexpr (SCORE) {
      if (score_live && tb < score_end) {
        // Sp sub-tiles: logit_prev(head 4*grp + r, key tb + 16*st + col); heads 8..15 are padding.
        float tot[4];
        auto head_reduce = [&](auto is_max) {
          constexpr bool MAX = decltype(is_max)::value;
#pragma unroll
          for (int st = 0; st < 4; ++st) {
            f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
            acc = mfma16x16x32(qp0, as_bf16x8(X.k[st][0]), acc);
            acc = mfma16x16x32(qp1, as_bf16x8(X.k[st][1]), acc);
            const float u0 = fast_exp2(fmaf(acc[0], a.scale2, -pn[0]));
            const float u1 = fast_exp2(fmaf(acc[1], a.scale2, -pn[1]));
            const float u2 = fast_exp2(fmaf(acc[2], a.scale2, -pn[2]));
            const float u3 = fast_exp2(fmaf(acc[3], a.scale2, -pn[3]));
            // Combine head halves 0-3 (group 0) and 4-7 (group 1); groups 2, 3 carry padding.
            tot[st] = MAX ? xor16_max(fmaxf(fmaxf(u0, u1), fmaxf(u2, u3))) : xor16_sum((u0 + u1) + (u2 + u3));
          }
        };
        if (max_mode)
          head_reduce(std::true_type{});
        else
          head_reduce(std::false_type{});
        // Lanes < 32 hold every sub-tile's totals; lane l owns key tb + l (sub-tile l/16, column l%16).
        const float send = grp == 0 ? tot[2] : tot[3];
        const float recv = lane_xor32(send);
        const float val = grp == 0 ? tot[0] : (grp == 1 ? tot[1] : recv);
        if (tb + lane < score_end) srow[int64_t(own_slot(X)) * a.scores_ss] = X.osc + val;
      }
    }
  };

  // Pipeline: slots two tiles ahead, rows and old scores one tile ahead. The K/V
  // buffers alternate between A and B, so no register copies are needed.
  Tile A, B;
  int32_t s_ahead[4];
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    A.s[st] = slot_at(k0 + 16 * st + col);
    B.s[st] = slot_at(k0 + TILE + 16 * st + col);
  }
  A.osc = B.osc = 0.f;
  issue_rows(A);
  auto step = [&](int t, Tile& X, Tile& Y) {
    const int64_t tb = k0 + int64_t(t) * TILE;
    // Past the last tile the slots are 0: the null slot's rows are loaded (one cached line per
    // wave) instead of branching around the loads.
#pragma unroll
    for (int st = 0; st < 4; ++st) s_ahead[st] = slot_at(tb + 2 * TILE + 16 * st + col);
    issue_rows(Y);
    // Keep the loads above the compute: the scheduler would otherwise sink them below it and
    // expose their latency at the next step.
    __builtin_amdgcn_sched_barrier(0);
    compute(t, X);
#pragma unroll
    for (int st = 0; st < 4; ++st) X.s[st] = s_ahead[st];
  };
  for (int t = 0; t < ntiles; t += 2) {
    step(t, A, B);
    if (t + 1 < ntiles) step(t + 1, B, A);
  }

  if constexpr (ATTN) {
    if (k0 < attn_end) {
      const float lt = xor32_sum(xor16_sum(l_run));
      if (col < GROUP) {
        float* pp = a.part + ((int64_t(b) * a.max_splits + split) * a.q_heads + hq) * PART;
#pragma unroll
        for (int j = 0; j < 4; ++j) *reinterpret_cast<f32x4_t*>(pp + 16 * j + 4 * grp) = oacc[j];
        if (grp == 0) {
          pp[D] = m_run;
          pp[D + 1] = lt;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Fused attention kernel over a balanced partition of the batch's keys.
//
// The batch's resident keys form one global range [0, T), T = indptr[bs] (the
// CSR concatenates the sequences). Workgroup w of P takes [w*C, (w+1)*C) with
// C = ceil(T / P), so every workgroup streams the same number of keys whatever
// the sequence lengths; its range splits into segments at sequence ends, and
// each segment leaves one attention partial, slot (w + b) of the partial buffer
// (w + b is unique: a later workgroup never starts in an earlier sequence).
//
// Per 64-key tile a wave (one KV head) computes one S^T = K . [Qcur | Qpend]^T
// tile per 16 keys with v_mfma_f32_16x16x32_bf16: columns 0-7 are the current
// query's 8 heads (attention), columns 8-15 the pending query's 8 heads (the
// lagged score update, whose normaliser is known since the previous call).
// O^T += V^T . P^T takes V transposed through LDS (ds_read_b64_tr_b16); the
// pending columns' probabilities are summed (or maxed) over heads through a
// 2 KiB LDS transpose and added to the keys' scores.
// ---------------------------------------------------------------------------
constexpr int FUSED_THREADS = 64 * MAX_KVH;

struct FusedArgs {
  const uint16_t* q;
  int64_t q_sb, q_sh;
  const uint16_t* k;
  const uint16_t* v;
  int64_t kv_ss, kv_sh;
  const int32_t* indptr;
  const void* indices;
  const int32_t* mode;
  const void* rows;
  int rows_dtype;
  float* scores;
  int64_t scores_sg, scores_ss;
  const uint16_t* pq;   // pending queries [rows, q_heads, D] (LAG)
  const float* pnorm;   // pending normalisers [rows, q_heads]
  const int32_t* plen;  // pending list lengths [rows]
  float* part;          // [P + bs, q_heads, PART]
  int bs, q_heads, kv_heads;
  int combined;  // scores laid out [slot][8 heads] (head stride 1, slot stride 8), 8 KV heads
  float scale2;  // sm_scale * log2(e)
};

// Keys per workgroup for P workgroups over T keys (0 when T == 0).
GSE_DEVICE int64_t fused_chunk(int64_t T, int P) { return (T + P - 1) / P; }

// Largest b in [0, bs) with indptr[b] <= p (indptr non-decreasing, indptr[0] = 0 <= p).
GSE_DEVICE int seq_of(const int32_t* indptr, int bs, int64_t p) {
  int lo = 0, hi = bs - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (int64_t(indptr[mid]) <= p) lo = mid; else hi = mid - 1;
  }
  return lo;
}

template <bool LAG, typename IdxT>
__global__ __launch_bounds__(FUSED_THREADS) void decode_fused_kernel(FusedArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t vtile[MAX_KVH][TILE * LDS_ROW];
  __shared__ __attribute__((aligned(16))) float sbuf[LAG ? MAX_KVH : 1][LAG ? GROUP * TILE : 4];
  // Per-tile score totals of every KV head ([tile parity][head][key]) for the combined update.
  __shared__ float wsum[LAG ? 2 : 1][LAG ? MAX_KVH : 1][LAG ? TILE + 4 : 4];

  const int lane = threadIdx.x & 63;
  const int g = threadIdx.x >> 6;
  if (g >= a.kv_heads) return;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const bool cur = col < GROUP;  // column holds a current-query head (else a pending one)
  const int hq = g * GROUP + (col & 7);

  // Key positions are CSR offsets (int32 in the CSR itself).
  const int P = gridDim.x;
  const int w = blockIdx.x;
  const int T = a.indptr[a.bs];
  const int C = int(fused_chunk(T, P));
  int p = w * C;
  const int p_end = p + C < T ? p + C : T;
  if (p >= p_end) return;
  int b = seq_of(a.indptr, a.bs, p);

  const uint16_t* kbase = a.k + int64_t(g) * a.kv_sh + 8 * grp;
  const uint16_t* vbase = a.v + int64_t(g) * a.kv_sh + 8 * grp;
  const uint64_t kv_row = uint64_t(a.kv_ss);  // elements per slot
  uint16_t* vt = vtile[g];
  float* sb = sbuf[LAG ? g : 0];
  float* srow = a.scores + int64_t(g) * a.scores_sg;
  const IdxT* idx = static_cast<const IdxT*>(a.indices);

  // Combined score update: wave g reads and writes the 8 heads' scores of keys 8g..8g+7 of a
  // tile, 16 bytes per lane (lanes 0-15), so each slot's 32-byte score row moves once.
  const int l16 = lane & 15;
  const int wkey = 8 * g + (l16 >> 1);  // this lane's key in the tile
  const int whead = 4 * (l16 & 1);      // first of its 4 heads

  struct Tile {
    int32_t s[4];
    uint4 k[4][2], v[4][2];
    f32x4_t osc;  // old scores: own key (per-head path) or 4 heads of key wkey (combined)
    int32_t os;   // slot of key wkey (combined)
  };

  while (p < p_end) {
    while (a.indptr[b + 1] <= p) ++b;  // skip empty sequences
    const int seq_start = a.indptr[b];
    const int seq_end = a.indptr[b + 1];
    const int s0 = p;
    const int s1 = seq_end < p_end ? seq_end : p_end;
    const int64_t row = load_index_dyn(a.rows, a.rows_dtype, b);

    // Pending score of this row: keys [seq_start, score_end) of the list get it.
    int score_end = s0;
    bool max_mode = false;
    if constexpr (LAG) {
      const int md = a.mode[row];
      const int pl = a.plen[row];
      if ((md == 1 || md == 2) && pl > 0) {
        score_end = seq_start + pl < s1 ? seq_start + pl : s1;
        max_mode = md == 2;
      }
    }
    const bool seg_scores = LAG && score_end > s0;

    // B operand: column col supplies dims [8*grp, 8*grp + 8) and [32 + 8*grp, ...) of its head.
    bf16x8_t qf0 = {}, qf1 = {};
    float sub = -INFINITY;  // the exponent's reference: running max (current) or pending normaliser
    if (cur) {
      const uint16_t* qp = a.q + int64_t(b) * a.q_sb + int64_t(hq) * a.q_sh + 8 * grp;
      qf0 = as_bf16x8(ld16(qp));
      qf1 = as_bf16x8(ld16(qp + 32));
    } else if (seg_scores) {
      const uint16_t* qp = a.pq + (row * a.q_heads + hq) * D + 8 * grp;
      qf0 = as_bf16x8(ld16(qp));
      qf1 = as_bf16x8(ld16(qp + 32));
      sub = a.pnorm[row * a.q_heads + hq] * kLog2e;
    } else {
      sub = INFINITY;  // no pending score: its probabilities are exactly 0
    }
    float l_run = 0.f;
    f32x4_t oacc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) oacc[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // Slot of global key i (slot 0, the null slot, past the segment); the index load is
    // issued for every lane so every path issues the same loads.
    auto slot_at = [&](int i) -> int32_t {
      const int32_t s = int32_t(idx[i < s1 ? i : s1 - 1]);
      return i < s1 ? s : 0;
    };
    auto own_slot = [&](const Tile& X) -> int32_t {
      return grp == 0 ? X.s[0] : (grp == 1 ? X.s[1] : (grp == 2 ? X.s[2] : X.s[3]));
    };
    auto issue_rows = [&](Tile& X) {
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const uint64_t off = uint64_t(uint32_t(X.s[st])) * kv_row;
        X.k[st][0] = ld16(kbase + off);
        X.k[st][1] = ld16(kbase + off + 32);
        X.v[st][0] = ld16(vbase + off);
        X.v[st][1] = ld16(vbase + off + 32);
      }
      if constexpr (LAG) {
        if (a.combined) {
          const int32_t sv = (g >> 1) == 0 ? X.s[0] : ((g >> 1) == 1 ? X.s[1] : ((g >> 1) == 2 ? X.s[2] : X.s[3]));
          X.os = __shfl(sv, 8 * (g & 1) + (l16 >> 1), kWave);
          X.osc = *reinterpret_cast<const f32x4_t*>(a.scores + uint64_t(uint32_t(X.os)) * GROUP + whead);
        } else {
          X.osc[0] = srow[uint64_t(uint32_t(own_slot(X))) * a.scores_ss];
        }
      }
    };

    auto compute = [&](int t, Tile& X) {
      const int tb = s0 + t * TILE;
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        *reinterpret_cast<uint4*>(vt + (16 * st + col) * LDS_ROW + 8 * grp) = X.v[st][0];
        *reinterpret_cast<uint4*>(vt + (16 * st + col) * LDS_ROW + 32 + 8 * grp) = X.v[st][1];
      }
      // sc[st][r]: logit (unscaled) of key tb + 16*st + 4*grp + r against column col.
      f32x4_t sc[4];
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
        acc = mfma16x16x32(as_bf16x8(X.k[st][0]), qf0, acc);
        sc[st] = mfma16x16x32(as_bf16x8(X.k[st][1]), qf1, acc);
      }
      if (tb + TILE > s1) {  // the segment's last tile: keys past its end take no mass
        const int lim = s1 - tb;
#pragma unroll
        for (int st = 0; st < 4; ++st)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (16 * st + 4 * grp + r >= lim) sc[st][r] = -INFINITY;
      }
      float tmax = fmaxf(fmaxf(fmaxf(sc[0][0], sc[0][1]), fmaxf(sc[0][2], sc[0][3])),
                         fmaxf(fmaxf(sc[1][0], sc[1][1]), fmaxf(sc[1][2], sc[1][3])));
      tmax = fmaxf(tmax, fmaxf(fmaxf(fmaxf(sc[2][0], sc[2][1]), fmaxf(sc[2][2], sc[2][3])),
                               fmaxf(fmaxf(sc[3][0], sc[3][1]), fmaxf(sc[3][2], sc[3][3]))));
      tmax = xor32_max(xor16_max(tmax)) * a.scale2;  // log2 units (scale > 0)
      // Lazy rescale of the current columns: keep the reference unless some head's tile
      // maximum exceeds it by more than 2^8 (exact: O and l share the reference).
      if (__any(cur && tmax > sub + 8.f)) {
        if (cur) {
          const float m_new = fmaxf(sub, tmax);
          const float corr = fast_exp2(sub - m_new);
          sub = m_new;
          l_run *= corr;
#pragma unroll
          for (int j = 0; j < 4; ++j) oacc[j] = oacc[j] * corr;
        }
      }
      float psum = 0.f;
#pragma unroll
      for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          sc[st][r] = fast_exp2(fmaf(sc[st][r], a.scale2, -sub));
          psum += sc[st][r];
        }
      l_run += psum;  // meaningful in the current columns only
      if constexpr (LAG) {
        // Pending columns: p of (key 16*st + 4*grp + r, head col - 8) -> sb[(col - 8) * 64 + key].
        if (seg_scores && !cur) {
#pragma unroll
          for (int st = 0; st < 4; ++st)
            *reinterpret_cast<f32x4_t*>(sb + (col - GROUP) * TILE + 16 * st + 4 * grp) = sc[st];
        }
      }
      // P^T operands: half 0 covers sub-tiles 0/1, half 1 sub-tiles 2/3; k-element e maps to
      // sub-tile 2*half + e/4, key 4*grp + e%4.
      uint4 pa, pb;
      pa.x = pack_bf16x2(sc[0][0], sc[0][1]);
      pa.y = pack_bf16x2(sc[0][2], sc[0][3]);
      pa.z = pack_bf16x2(sc[1][0], sc[1][1]);
      pa.w = pack_bf16x2(sc[1][2], sc[1][3]);
      pb.x = pack_bf16x2(sc[2][0], sc[2][1]);
      pb.y = pack_bf16x2(sc[2][2], sc[2][3]);
      pb.z = pack_bf16x2(sc[3][0], sc[3][1]);
      pb.w = pack_bf16x2(sc[3][2], sc[3][3]);
      __builtin_amdgcn_wave_barrier();
      // Lanes of group grp read the V^T fragments of keys 32*half + 16*h + 4*grp + e at dims
      // 16*j + 4*(lane%4) (ds_read_b64_tr_b16).
      const uint16_t* vr = vt + (4 * grp + ((lane & 15) >> 2)) * LDS_ROW + 4 * (lane & 3);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const s16x4_t a0 = ds_read_tr16(vr + 16 * j);
        const s16x4_t a1 = ds_read_tr16(vr + 16 * LDS_ROW + 16 * j);
        const s16x4_t b0 = ds_read_tr16(vr + 32 * LDS_ROW + 16 * j);
        const s16x4_t b1 = ds_read_tr16(vr + 48 * LDS_ROW + 16 * j);
        oacc[j] = mfma16x16x32(join_bf16x8(a0, a1), as_bf16x8(pa), oacc[j]);
        oacc[j] = mfma16x16x32(join_bf16x8(b0, b1), as_bf16x8(pb), oacc[j]);
      }
      if constexpr (LAG) {
        if (seg_scores && tb < score_end) {
          // Lane l owns key tb + l: its 8 heads' probabilities, summed or maxed.
          float tot = sb[lane];
          if (max_mode) {
#pragma unroll
            for (int h = 1; h < GROUP; ++h) tot = fmaxf(tot, sb[h * TILE + lane]);
          } else {
#pragma unroll
            for (int h = 1; h < GROUP; ++h) tot += sb[h * TILE + lane];
          }
          if (a.combined) {
            // Every head's totals meet in LDS (all waves work on the same tile), then each
            // slot's row of 8 scores is written once.
            wsum[t & 1][g][lane] = tot;
            __syncthreads();
            const f32x4_t add = {wsum[t & 1][whead][wkey], wsum[t & 1][whead + 1][wkey],
                                 wsum[t & 1][whead + 2][wkey], wsum[t & 1][whead + 3][wkey]};
            if (lane < 16 && tb + wkey < score_end)
              *reinterpret_cast<f32x4_t*>(a.scores + uint64_t(uint32_t(X.os)) * GROUP + whead) = X.osc + add;
          } else if (tb + lane < score_end) {
            srow[uint64_t(uint32_t(own_slot(X))) * a.scores_ss] = X.osc[0] + tot;
          }
        }
      }
      __builtin_amdgcn_wave_barrier();
    };

    const int ntiles = (s1 - s0 + TILE - 1) / TILE;
    Tile A, B;
    int32_t s_ahead[4];
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      A.s[st] = slot_at(s0 + 16 * st + col);
      B.s[st] = slot_at(s0 + TILE + 16 * st + col);
    }
    A.osc = B.osc = f32x4_t{0.f, 0.f, 0.f, 0.f};
    A.os = B.os = 0;
    issue_rows(A);
    // Per step: slots two tiles ahead and rows one tile ahead are issued before the compute.
    // Past the segment the slots are 0 and the null slot's rows are loaded (cached lines)
    // instead of branching around the loads.
    auto step = [&](int t, Tile& X, Tile& Y) {
      const int tb = s0 + t * TILE;
#pragma unroll
      for (int st = 0; st < 4; ++st) s_ahead[st] = slot_at(tb + 2 * TILE + 16 * st + col);
      issue_rows(Y);
      __builtin_amdgcn_sched_barrier(0);
      compute(t, X);
#pragma unroll
      for (int st = 0; st < 4; ++st) X.s[st] = s_ahead[st];
    };
    // Both steps in every iteration, the odd last tile peeled: no path through the loop
    // skips a step's loads, so the compiler's wait counts stay exact.
    int t = 0;
    for (; t + 1 < ntiles; t += 2) {
      step(t, A, B);
      step(t + 1, B, A);
    }
    if (t < ntiles) step(t, A, B);

    // This segment's partial: O^T rows 4*grp + r of dim block j, column col; m and l.
    const float lt = xor32_sum(xor16_sum(l_run));
    if (cur) {
      float* pp = a.part + ((int64_t(w) + b) * a.q_heads + hq) * PART;
#pragma unroll
      for (int j = 0; j < 4; ++j) *reinterpret_cast<f32x4_t*>(pp + 16 * j + 4 * grp) = oacc[j];
      if (grp == 0) {
        pp[D] = sub;
        pp[D + 1] = lt;
      }
    }
    p = s1;
    ++b;
  }
}

struct MergeArgs {
  const float* part;
  const int32_t* indptr;
  const void* sinks;
  int sinks_dtype;
  uint16_t* o;
  int64_t o_sb, o_sh;
  float* norm_out;  // [bs, q_heads]
  // Pending update (LAG): pq[row] <- q[b], pnorm[row] <- norm, plen[row] <- len (0 if mode not 1/2).
  const uint16_t* q;
  int64_t q_sb, q_sh;
  const int32_t* mode;
  const void* rows;
  int rows_dtype;
  uint16_t* pq;
  float* pnorm;
  int32_t* plen;
  int bs, q_heads, nparts;  // nparts = P, the fused kernel's workgroup count
};

// Grid (bs): thread (head t/8, dims [8*(t%8), +8)) merges the partials of its head with
// the sink: o = sum_w 2^(m_w - M) o_w / (2^(sink - M) + sum_w 2^(m_w - M) l_w).
__global__ __launch_bounds__(512) void decode_merge_kernel(MergeArgs a) {
  const int b = blockIdx.x;
  const int h = threadIdx.x >> 3;
  const int j = threadIdx.x & 7;
  if (h >= a.q_heads) return;
  const int64_t T = a.indptr[a.bs];
  const int64_t C = fused_chunk(T, a.nparts);
  const int64_t start = a.indptr[b], end = a.indptr[b + 1];
  int64_t wf = 1, wl = 0;
  if (end > start) {
    wf = start / C;
    wl = (end - 1) / C;
  }
  const float sink2 = load_float_dyn(a.sinks, a.sinks_dtype, h) * kLog2e;
  float mx = sink2;
  for (int64_t w = wf; w <= wl; ++w) mx = fmaxf(mx, a.part[((w + b) * a.q_heads + h) * PART + D]);
  float lsum = fast_exp2(sink2 - mx);
  f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  for (int64_t w = wf; w <= wl; ++w) {
    const float* ps = a.part + ((w + b) * a.q_heads + h) * PART;
    const float wt = fast_exp2(ps[D] - mx);
    lsum += wt * ps[D + 1];
    acc0 += wt * *reinterpret_cast<const f32x4_t*>(ps + 8 * j);
    acc1 += wt * *reinterpret_cast<const f32x4_t*>(ps + 8 * j + 4);
  }
  const float inv = 1.f / lsum;
  uint4 out;
  out.x = pack_bf16x2(acc0[0] * inv, acc0[1] * inv);
  out.y = pack_bf16x2(acc0[2] * inv, acc0[3] * inv);
  out.z = pack_bf16x2(acc1[0] * inv, acc1[1] * inv);
  out.w = pack_bf16x2(acc1[2] * inv, acc1[3] * inv);
  *reinterpret_cast<uint4*>(a.o + int64_t(b) * a.o_sb + int64_t(h) * a.o_sh + 8 * j) = out;
  const float norm = (mx + __log2f(lsum)) * kLn2;
  if (j == 0) a.norm_out[int64_t(b) * a.q_heads + h] = norm;
  if (a.pq) {
    const int64_t row = load_index_dyn(a.rows, a.rows_dtype, b);
    const int md = a.mode[row];
    const bool live = md == 1 || md == 2;
    if (live) {
      *reinterpret_cast<uint4*>(a.pq + (row * a.q_heads + h) * D + 8 * j) =
          *reinterpret_cast<const uint4*>(a.q + int64_t(b) * a.q_sb + int64_t(h) * a.q_sh + 8 * j);
      if (j == 0) a.pnorm[row * a.q_heads + h] = norm;
    }
    if (threadIdx.x == 0) a.plen[row] = live ? int32_t(end - start) : 0;
  }
}

struct NormArgs {
  const float* lse;
  int64_t lse_sb, lse_sh;
  const int32_t* num_splits;
  const int32_t* indptr;
  const void* sinks;
  int sinks_dtype;
  float* norm;  // [bs, q_heads]
  int q_heads, max_kv_splits, min_kv;
};

// R:180-188: the normaliser from SGLang's split log-sum-exps, started at (sink, 1).
__global__ void norm_from_lse_kernel(NormArgs a) {
  const int b = blockIdx.x;
  const int h = threadIdx.x;
  if (h >= a.q_heads) return;
  const int64_t len = int64_t(a.indptr[b + 1]) - a.indptr[b];
  const int64_t splits = a.num_splits[b];
  const int64_t per = ((len + splits - 1) / splits + a.min_kv - 1) / a.min_kv * a.min_kv;
  float m = load_float_dyn(a.sinks, a.sinks_dtype, h);
  float s = 1.f;
  for (int i = 0; i < a.max_kv_splits; ++i) {
    if (int64_t(i) * per < len) {
      const float x = a.lse[int64_t(b) * a.lse_sb + int64_t(h) * a.lse_sh + i];
      const float n = fmaxf(m, x);
      s = s * expf(m - n) + expf(x - n);
      m = n;
    }
  }
  a.norm[int64_t(b) * a.q_heads + h] = m + logf(s);
}

__global__ void clear_pending_kernel(const void* rows, int rows_dtype, int n_rows, int32_t* plen) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n_rows) plen[load_index_dyn(rows, rows_dtype, i)] = 0;
}

}  // namespace gse

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
#include "host.hpp"

using namespace gse;

namespace {

// Workgroups of the fused kernel: one per compute unit of the current device (cached).
int fused_workgroups() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

}  // namespace

extern "C" int64_t gse_decode_workspace_bytes(int bs, int max_splits, int q_heads, int head_dim) {
  // Fused-kernel partials (one per workgroup-sequence segment: at most P + bs of them) and
  // the per-head normalisers; the score-only pass of GSE_SCORE_EAGER needs nothing more.
  (void)max_splits;
  const int64_t parts = int64_t(fused_workgroups()) + bs;
  return parts * q_heads * (head_dim + 4) * int64_t(sizeof(float)) + int64_t(bs) * q_heads * 4;
}

namespace {

int check_decode_shape(int q_heads, int kv_heads, int head_dim, int chunk, int max_splits) {
  if (head_dim != D) return gse_fail(GSE_ESHAPE, "decode: head_dim must be 64");
  if (kv_heads < 1 || kv_heads > MAX_KVH || q_heads != GROUP * kv_heads)
    return gse_fail(GSE_ESHAPE, "decode: need q_heads == 8 * kv_heads and 1 <= kv_heads <= 8");
  if (chunk < TILE || chunk % TILE) return gse_fail(GSE_EINVAL, "decode: chunk must be a positive multiple of 64");
  if (max_splits < 1 || max_splits > 65535) return gse_fail(GSE_EINVAL, "decode: max_splits out of range");
  return GSE_OK;
}

template <bool ATTN, bool SCORE, bool ROWVIEW>
int launch_split(const DecodeArgs& a, int indices_dtype, int nblocks_y, hipStream_t s) {
  dim3 grid(a.max_splits, nblocks_y), block(64 * MAX_KVH);
  if (nblocks_y == 0) return GSE_OK;
  if (indices_dtype == GSE_I64)
    hipLaunchKernelGGL((decode_split_kernel<ATTN, SCORE, ROWVIEW, int64_t>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((decode_split_kernel<ATTN, SCORE, ROWVIEW, int32_t>), grid, block, 0, s, a);
  return gse_launch_check("decode_split");
}

}  // namespace

extern "C" int gse_decode(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                          const void* k_pool, const void* v_pool, int64_t kv_stride_s, int64_t kv_stride_h,
                          const int32_t* kv_indptr, const void* kv_indices, int indices_dtype,
                          const void* sinks, int sinks_dtype, const int32_t* mode_by_row, const void* rows,
                          int rows_dtype, float* scores, int64_t scores_stride_g, int64_t scores_stride_s,
                          void* o, int64_t o_stride_b, int64_t o_stride_h, float* norm_out,
                          void* pend_q, float* pend_norm, int32_t* pend_len,
                          int bs, int q_heads, int kv_heads, int head_dim, float sm_scale, int chunk,
                          int max_splits, int score_mode, void* workspace, int64_t workspace_bytes,
                          gse_stream_t stream) {
  if (int rc = check_decode_shape(q_heads, kv_heads, head_dim, chunk, max_splits)) return rc;
  if (bs < 0) return gse_fail(GSE_EINVAL, "decode: bs < 0");
  if (bs == 0) return GSE_OK;
  if (workspace_bytes < gse_decode_workspace_bytes(bs, max_splits, q_heads, head_dim))
    return gse_fail(GSE_EWORKSPACE, "decode: workspace too small");
  if (!q || !k_pool || !v_pool || !kv_indptr || !kv_indices || !sinks || !o)
    return gse_fail(GSE_EINVAL, "decode: null pointer");
  if (score_mode != GSE_SCORE_NONE && (!mode_by_row || !rows || !scores))
    return gse_fail(GSE_EINVAL, "decode: scoring needs mode, rows and scores");
  if (score_mode == GSE_SCORE_LAG && (!pend_q || !pend_norm || !pend_len))
    return gse_fail(GSE_EINVAL, "decode: LAG mode needs pending buffers");
  if (score_mode < GSE_SCORE_NONE || score_mode > GSE_SCORE_LAG) return gse_fail(GSE_EINVAL, "decode: bad score_mode");
  if ((q_stride_h % 8) || (q_stride_b % 8) || (kv_stride_s % 8) || (kv_stride_h % 8) || (o_stride_b % 8) ||
      (o_stride_h % 8))
    return gse_fail(GSE_EINVAL, "decode: strides must be multiples of 8 elements (16-byte rows)");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);

  const int P = fused_workgroups();
  float* part = static_cast<float*>(workspace);
  float* norm_ws = part + (int64_t(P) + bs) * q_heads * PART;
  float* norm = norm_out ? norm_out : norm_ws;

  FusedArgs f = {};
  f.q = static_cast<const uint16_t*>(q);
  f.q_sb = q_stride_b;
  f.q_sh = q_stride_h;
  f.k = static_cast<const uint16_t*>(k_pool);
  f.v = static_cast<const uint16_t*>(v_pool);
  f.kv_ss = kv_stride_s;
  f.kv_sh = kv_stride_h;
  f.indptr = kv_indptr;
  f.indices = kv_indices;
  f.mode = mode_by_row;
  f.rows = rows;
  f.rows_dtype = rows_dtype;
  f.scores = scores;
  f.scores_sg = scores_stride_g;
  f.scores_ss = scores_stride_s;
  f.part = part;
  f.bs = bs;
  f.q_heads = q_heads;
  f.kv_heads = kv_heads;
  f.scale2 = sm_scale * kLog2e;

  MergeArgs m = {};
  m.part = part;
  m.indptr = kv_indptr;
  m.sinks = sinks;
  m.sinks_dtype = sinks_dtype;
  m.o = static_cast<uint16_t*>(o);
  m.o_sb = o_stride_b;
  m.o_sh = o_stride_h;
  m.norm_out = norm;
  m.q = f.q;
  m.q_sb = q_stride_b;
  m.q_sh = q_stride_h;
  m.mode = mode_by_row;
  m.rows = rows;
  m.rows_dtype = rows_dtype;
  m.bs = bs;
  m.q_heads = q_heads;
  m.nparts = P;

  const bool lag = score_mode == GSE_SCORE_LAG;
  f.combined = kv_heads == MAX_KVH && scores_stride_g == 1 && scores_stride_s == GROUP &&
               (reinterpret_cast<uintptr_t>(scores) & 15) == 0;
  if (lag) {
    f.pq = static_cast<const uint16_t*>(pend_q);
    f.pnorm = pend_norm;
    f.plen = pend_len;
    m.pq = static_cast<uint16_t*>(pend_q);
    m.pnorm = pend_norm;
    m.plen = pend_len;
  }
  const dim3 grid(P), block(FUSED_THREADS);
  if (indices_dtype == GSE_I64) {
    if (lag)
      hipLaunchKernelGGL((decode_fused_kernel<true, int64_t>), grid, block, 0, s, f);
    else
      hipLaunchKernelGGL((decode_fused_kernel<false, int64_t>), grid, block, 0, s, f);
  } else {
    if (lag)
      hipLaunchKernelGGL((decode_fused_kernel<true, int32_t>), grid, block, 0, s, f);
    else
      hipLaunchKernelGGL((decode_fused_kernel<false, int32_t>), grid, block, 0, s, f);
  }
  int rc = gse_launch_check("decode_fused");
  if (rc) return rc;
  hipLaunchKernelGGL(decode_merge_kernel, dim3(bs), dim3(512), 0, s, m);
  if ((rc = gse_launch_check("decode_merge"))) return rc;
  if (score_mode == GSE_SCORE_EAGER) {
    // This step's scores need its final normaliser: a second, score-only pass over K.
    DecodeArgs a = {};
    a.k = f.k;
    a.v = f.k;
    a.kv_ss = kv_stride_s;
    a.kv_sh = kv_stride_h;
    a.src.indptr = kv_indptr;
    a.src.indices = kv_indices;
    a.mode = mode_by_row;
    a.rows = rows;
    a.rows_dtype = rows_dtype;
    a.scores = scores;
    a.scores_sg = scores_stride_g;
    a.scores_ss = scores_stride_s;
    a.sq = f.q;
    a.sq_sb = q_stride_b;
    a.sq_sh = q_stride_h;
    a.snorm = norm;
    a.snorm_sb = q_heads;
    a.slen = nullptr;
    a.score_by_row = 0;
    a.q_heads = q_heads;
    a.kv_heads = kv_heads;
    a.chunk = chunk;
    a.max_splits = max_splits;
    a.scale2 = sm_scale * kLog2e;
    if ((rc = launch_split<false, true, false>(a, indices_dtype, bs, s))) return rc;
  }
  return GSE_OK;
}

extern "C" int gse_decode_flush(const void* k_pool, int64_t kv_stride_s, int64_t kv_stride_h,
                                const int32_t* table, int64_t table_stride, const int32_t* req_to_token,
                                int64_t r2t_stride, int64_t r2t_width, const int32_t* frontier, const int32_t* count,
                                const int32_t* mode_by_row, const void* rows, int rows_dtype, int n_rows,
                                float* scores, int64_t scores_stride_g, int64_t scores_stride_s, void* pend_q,
                                float* pend_norm,
                                int32_t* pend_len, int q_heads, int kv_heads, int head_dim, float sm_scale,
                                int chunk, int max_splits, gse_stream_t stream) {
  if (int rc = check_decode_shape(q_heads, kv_heads, head_dim, chunk, max_splits)) return rc;
  if (n_rows <= 0) return n_rows < 0 ? gse_fail(GSE_EINVAL, "flush: n_rows < 0") : GSE_OK;
  if (!k_pool || !table || !req_to_token || !frontier || !count || !mode_by_row || !rows || !scores || !pend_q ||
      !pend_norm || !pend_len)
    return gse_fail(GSE_EINVAL, "flush: null pointer");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  DecodeArgs a = {};
  a.k = static_cast<const uint16_t*>(k_pool);
  a.v = a.k;
  a.kv_ss = kv_stride_s;
  a.kv_sh = kv_stride_h;
  a.src.table = table;
  a.src.table_stride = table_stride;
  a.src.r2t = req_to_token;
  a.src.r2t_stride = r2t_stride;
  a.src.r2t_width = r2t_width;
  a.src.frontier = frontier;
  a.src.count = count;
  a.mode = mode_by_row;
  a.rows = rows;
  a.rows_dtype = rows_dtype;
  a.scores = scores;
  a.scores_sg = scores_stride_g;
  a.scores_ss = scores_stride_s;
  a.sq = static_cast<const uint16_t*>(pend_q);
  a.sq_sb = int64_t(q_heads) * D;
  a.sq_sh = D;
  a.snorm = pend_norm;
  a.snorm_sb = q_heads;
  a.slen = pend_len;
  a.score_by_row = 1;
  a.q_heads = q_heads;
  a.kv_heads = kv_heads;
  a.chunk = chunk;
  a.max_splits = max_splits;
  a.scale2 = sm_scale * kLog2e;
  int rc = launch_split<false, true, true>(a, GSE_I32, n_rows, s);
  if (rc) return rc;
  hipLaunchKernelGGL(clear_pending_kernel, dim3((n_rows + 255) / 256), dim3(256), 0, s, rows, rows_dtype, n_rows,
                     pend_len);
  return gse_launch_check("clear_pending");
}

extern "C" int gse_decode_scores_from_lse(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                          const void* k_pool, int64_t kv_stride_s, int64_t kv_stride_h,
                                          const int32_t* kv_indptr, const void* kv_indices, int indices_dtype,
                                          const float* attn_lse, int64_t lse_stride_b, int64_t lse_stride_h,
                                          const int32_t* num_kv_splits, int max_kv_splits, int min_block_kv,
                                          const void* sinks, int sinks_dtype, const int32_t* mode_by_row,
                                          const void* rows, int rows_dtype, float* scores,
                                          int64_t scores_stride_g, int64_t scores_stride_s, int bs, int q_heads,
                                          int kv_heads,
                                          int head_dim, float sm_scale, int chunk, int max_splits, void* workspace,
                                          int64_t workspace_bytes, gse_stream_t stream) {
  if (int rc = check_decode_shape(q_heads, kv_heads, head_dim, chunk, max_splits)) return rc;
  if (bs <= 0) return bs < 0 ? gse_fail(GSE_EINVAL, "scores_from_lse: bs < 0") : GSE_OK;
  if (workspace_bytes < int64_t(bs) * q_heads * 4) return gse_fail(GSE_EWORKSPACE, "scores_from_lse: workspace");
  if (max_kv_splits < 1 || min_block_kv < 1) return gse_fail(GSE_EINVAL, "scores_from_lse: split layout");
  if (!q || !k_pool || !kv_indptr || !kv_indices || !attn_lse || !num_kv_splits || !sinks || !mode_by_row || !rows ||
      !scores)
    return gse_fail(GSE_EINVAL, "scores_from_lse: null pointer");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  float* norm = static_cast<float*>(workspace);
  NormArgs n = {attn_lse, lse_stride_b, lse_stride_h, num_kv_splits, kv_indptr, sinks, sinks_dtype,
                norm, q_heads, max_kv_splits, min_block_kv};
  hipLaunchKernelGGL(norm_from_lse_kernel, dim3(bs), dim3(64), 0, s, n);
  if (int rc = gse_launch_check("norm_from_lse")) return rc;
  DecodeArgs a = {};
  a.k = static_cast<const uint16_t*>(k_pool);
  a.v = a.k;
  a.kv_ss = kv_stride_s;
  a.kv_sh = kv_stride_h;
  a.src.indptr = kv_indptr;
  a.src.indices = kv_indices;
  a.mode = mode_by_row;
  a.rows = rows;
  a.rows_dtype = rows_dtype;
  a.scores = scores;
  a.scores_sg = scores_stride_g;
  a.scores_ss = scores_stride_s;
  a.sq = static_cast<const uint16_t*>(q);
  a.sq_sb = q_stride_b;
  a.sq_sh = q_stride_h;
  a.snorm = norm;
  a.snorm_sb = q_heads;
  a.slen = nullptr;
  a.score_by_row = 0;
  a.q_heads = q_heads;
  a.kv_heads = kv_heads;
  a.chunk = chunk;
  a.max_splits = max_splits;
  a.scale2 = sm_scale * kLog2e;
  return launch_split<false, true, false>(a, indices_dtype, bs, s);
}
