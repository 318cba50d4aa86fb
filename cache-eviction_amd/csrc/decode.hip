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
#include "common.hpp"

namespace gse {

constexpr int D = 64;        // head_dim
constexpr int GROUP = 8;     // query heads per KV head
constexpr int TILE = 32;     // keys per inner iteration (two 16-key MFMA sub-tiles)
constexpr int MAX_KVH = 8;   // waves per workgroup
constexpr int LDS_ROW = D + 8;  // padded bf16 row of the V staging tile
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
  int64_t scores_sg;
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

  auto slot_at = [&](int64_t i) -> int64_t {
    return i < k_end ? fetch_slot<ROWVIEW, IdxT>(a.src, row, base, cnt, fr, i) : int64_t(0);
  };

  const int ntiles = int((k_end - k0 + TILE - 1) / TILE);
  int64_t s0 = slot_at(k0 + col), s1 = slot_at(k0 + 16 + col);
  uint4 ka0 = ld16(kbase + s0 * a.kv_ss), ka1 = ld16(kbase + s0 * a.kv_ss + 8);
  uint4 kb0 = ld16(kbase + s1 * a.kv_ss), kb1 = ld16(kbase + s1 * a.kv_ss + 8);
  uint4 va0 = {}, va1 = {}, vb0 = {}, vb1 = {};
  if constexpr (ATTN) {
    va0 = ld16(vbase + s0 * a.kv_ss);
    va1 = ld16(vbase + s0 * a.kv_ss + 8);
    vb0 = ld16(vbase + s1 * a.kv_ss);
    vb1 = ld16(vbase + s1 * a.kv_ss + 8);
  }

  for (int t = 0; t < ntiles; ++t) {
    const int64_t tb = k0 + int64_t(t) * TILE;
    // Prefetch the next tile's rows.
    const int64_t nb = tb + TILE;
    int64_t n0 = 0, n1 = 0;
    uint4 nka0 = {}, nka1 = {}, nkb0 = {}, nkb1 = {}, nva0 = {}, nva1 = {}, nvb0 = {}, nvb1 = {};
    if (t + 1 < ntiles) {
      n0 = slot_at(nb + col);
      n1 = slot_at(nb + 16 + col);
      nka0 = ld16(kbase + n0 * a.kv_ss);
      nka1 = ld16(kbase + n0 * a.kv_ss + 8);
      nkb0 = ld16(kbase + n1 * a.kv_ss);
      nkb1 = ld16(kbase + n1 * a.kv_ss + 8);
      if constexpr (ATTN) {
        nva0 = ld16(vbase + n0 * a.kv_ss);
        nva1 = ld16(vbase + n0 * a.kv_ss + 8);
        nvb0 = ld16(vbase + n1 * a.kv_ss);
        nvb1 = ld16(vbase + n1 * a.kv_ss + 8);
      }
    }

    if constexpr (ATTN) {
      if (tb < attn_end) {
        // Stage V rows [key][dim] for the transposed read.
        *reinterpret_cast<uint4*>(vt + col * LDS_ROW + 16 * grp) = va0;
        *reinterpret_cast<uint4*>(vt + col * LDS_ROW + 16 * grp + 8) = va1;
        *reinterpret_cast<uint4*>(vt + (16 + col) * LDS_ROW + 16 * grp) = vb0;
        *reinterpret_cast<uint4*>(vt + (16 + col) * LDS_ROW + 16 * grp + 8) = vb1;

        f32x4_t sa = {0.f, 0.f, 0.f, 0.f}, sb = {0.f, 0.f, 0.f, 0.f};
        sa = mfma16x16x32(as_bf16x8(ka0), qc0, sa);
        sa = mfma16x16x32(as_bf16x8(ka1), qc1, sa);
        sb = mfma16x16x32(as_bf16x8(kb0), qc0, sb);
        sb = mfma16x16x32(as_bf16x8(kb1), qc1, sb);
        // sa[r]: head col, key tb + 4*grp + r; sb[r]: key tb + 16 + 4*grp + r.
        float x[8];
        float tmax = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t ka = tb + 4 * grp + r, kb = tb + 16 + 4 * grp + r;
          x[r] = ka < attn_end ? sa[r] * a.scale2 : -INFINITY;
          x[4 + r] = kb < attn_end ? sb[r] * a.scale2 : -INFINITY;
          tmax = fmaxf(tmax, fmaxf(x[r], x[4 + r]));
        }
        tmax = wave_max_xor(tmax, 16);
        tmax = wave_max_xor(tmax, 32);
        const float m_new = fmaxf(m_run, tmax);
        const float corr = fast_exp2(m_run - m_new);
        m_run = m_new;
        float psum = 0.f;
        float p[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          p[e] = fast_exp2(x[e] - m_new);
          psum += p[e];
        }
        l_run = l_run * corr + psum;
        uint4 pk;
        pk.x = pack_bf16x2(p[0], p[1]);
        pk.y = pack_bf16x2(p[2], p[3]);
        pk.z = pack_bf16x2(p[4], p[5]);
        pk.w = pack_bf16x2(p[6], p[7]);
        const bf16x8_t pb = as_bf16x8(pk);
        __builtin_amdgcn_wave_barrier();
        // V^T fragment: dim (col + 16j), keys kappa(8*grp + e).
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint16_t* vc = vt + col + 16 * j;
          uint4 av;
          av.x = uint32_t(vc[(4 * grp + 0) * LDS_ROW]) | (uint32_t(vc[(4 * grp + 1) * LDS_ROW]) << 16);
          av.y = uint32_t(vc[(4 * grp + 2) * LDS_ROW]) | (uint32_t(vc[(4 * grp + 3) * LDS_ROW]) << 16);
          av.z = uint32_t(vc[(16 + 4 * grp + 0) * LDS_ROW]) | (uint32_t(vc[(16 + 4 * grp + 1) * LDS_ROW]) << 16);
          av.w = uint32_t(vc[(16 + 4 * grp + 2) * LDS_ROW]) | (uint32_t(vc[(16 + 4 * grp + 3) * LDS_ROW]) << 16);
          oacc[j] = oacc[j] * corr;
          oacc[j] = mfma16x16x32(as_bf16x8(av), pb, oacc[j]);
        }
        __builtin_amdgcn_wave_barrier();
      }
    }

    if constexpr (SCORE) {
      if (do_score && tb < score_end) {
        f32x4_t pa = {0.f, 0.f, 0.f, 0.f}, pbv = {0.f, 0.f, 0.f, 0.f};
        pa = mfma16x16x32(qp0, as_bf16x8(ka0), pa);
        pa = mfma16x16x32(qp1, as_bf16x8(ka1), pa);
        pbv = mfma16x16x32(qp0, as_bf16x8(kb0), pbv);
        pbv = mfma16x16x32(qp1, as_bf16x8(kb1), pbv);
        // pa[r]: head 4*grp + r, key tb + col; pbv[r]: key tb + 16 + col.
        float ta, tbv;
        if (grp < 2) {
          float ua[4], ub[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            ua[r] = fast_exp2(pa[r] * a.scale2 - pn[r]);
            ub[r] = fast_exp2(pbv[r] * a.scale2 - pn[r]);
          }
          if (max_mode) {
            ta = fmaxf(fmaxf(ua[0], ua[1]), fmaxf(ua[2], ua[3]));
            tbv = fmaxf(fmaxf(ub[0], ub[1]), fmaxf(ub[2], ub[3]));
          } else {
            ta = (ua[0] + ua[1]) + (ua[2] + ua[3]);
            tbv = (ub[0] + ub[1]) + (ub[2] + ub[3]);
          }
        } else {
          ta = 0.f;
          tbv = 0.f;
        }
        const float oa = __shfl_xor(ta, 16, kWave), ob = __shfl_xor(tbv, 16, kWave);
        if (max_mode) {
          ta = fmaxf(ta, oa);
          tbv = fmaxf(tbv, ob);
        } else {
          ta += oa;
          tbv += ob;
        }
        // Lane l < 32 owns key tb + l: sub-tile 0 for l < 16, sub-tile 1 for 16 <= l < 32.
        if (lane < 32) {
          const int64_t key = tb + lane;
          if (key < score_end) {
            const int64_t slot = lane < 16 ? s0 : s1;
            const float val = lane < 16 ? ta : tbv;
            srow[slot] = srow[slot] + val;
          }
        }
      }
    }

    s0 = n0;
    s1 = n1;
    ka0 = nka0; ka1 = nka1; kb0 = nkb0; kb1 = nkb1;
    va0 = nva0; va1 = nva1; vb0 = nvb0; vb1 = nvb1;
  }

  if constexpr (ATTN) {
    if (k0 < attn_end) {
      float lt = wave_sum_xor(l_run, 16);
      lt = wave_sum_xor(lt, 32);
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

struct MergeArgs {
  const float* part;
  const int32_t* indptr;
  const void* sinks;
  int sinks_dtype;
  uint16_t* o;
  int64_t o_sb, o_sh;
  float* norm_out;  // [bs, q_heads] or null
  // Pending update (LAG): pq[row] <- q[b], pnorm[row] <- norm, plen[row] <- len (0 if mode not 1/2).
  const uint16_t* q;
  int64_t q_sb, q_sh;
  const int32_t* mode;
  const void* rows;
  int rows_dtype;
  uint16_t* pq;
  float* pnorm;
  int32_t* plen;
  int q_heads, chunk, max_splits;
};

// One workgroup per sequence; thread t handles head t/4, dims [16*(t%4), +16).
__global__ __launch_bounds__(256) void decode_merge_kernel(MergeArgs a) {
  const int b = blockIdx.x;
  const int h = threadIdx.x >> 2;
  const int dq = threadIdx.x & 3;
  if (h >= a.q_heads) return;
  const int64_t len = int64_t(a.indptr[b + 1]) - a.indptr[b];
  int nsplit = int((len + a.chunk - 1) / a.chunk);
  nsplit = nsplit < a.max_splits ? nsplit : a.max_splits;  // the host sizes chunk * max_splits >= len
  const float sink2 = load_float_dyn(a.sinks, a.sinks_dtype, h) * kLog2e;
  const float* pb = a.part + (int64_t(b) * a.max_splits * a.q_heads + h) * PART;
  const int64_t sstride = int64_t(a.q_heads) * PART;
  float mx = sink2;
  for (int s = 0; s < nsplit; ++s) mx = fmaxf(mx, pb[s * sstride + D]);
  float lsum = fast_exp2(sink2 - mx);
  float acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.f;
  for (int s = 0; s < nsplit; ++s) {
    const float* ps = pb + s * sstride;
    const float w = fast_exp2(ps[D] - mx);
    lsum += w * ps[D + 1];
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
      const f32x4_t v = *reinterpret_cast<const f32x4_t*>(ps + 16 * dq + i);
      acc[i] += w * v[0];
      acc[i + 1] += w * v[1];
      acc[i + 2] += w * v[2];
      acc[i + 3] += w * v[3];
    }
  }
  const float inv = 1.f / lsum;
  uint4 w0, w1;
  w0.x = pack_bf16x2(acc[0] * inv, acc[1] * inv);
  w0.y = pack_bf16x2(acc[2] * inv, acc[3] * inv);
  w0.z = pack_bf16x2(acc[4] * inv, acc[5] * inv);
  w0.w = pack_bf16x2(acc[6] * inv, acc[7] * inv);
  w1.x = pack_bf16x2(acc[8] * inv, acc[9] * inv);
  w1.y = pack_bf16x2(acc[10] * inv, acc[11] * inv);
  w1.z = pack_bf16x2(acc[12] * inv, acc[13] * inv);
  w1.w = pack_bf16x2(acc[14] * inv, acc[15] * inv);
  uint16_t* op = a.o + int64_t(b) * a.o_sb + int64_t(h) * a.o_sh + 16 * dq;
  *reinterpret_cast<uint4*>(op) = w0;
  *reinterpret_cast<uint4*>(op + 8) = w1;
  const float norm = (mx + __log2f(lsum)) * kLn2;
  if (a.norm_out && dq == 0) a.norm_out[int64_t(b) * a.q_heads + h] = norm;
  if (a.pq) {
    const int64_t row = load_index_dyn(a.rows, a.rows_dtype, b);
    const int md = a.mode[row];
    const bool live = md == 1 || md == 2;
    if (live) {
      const uint16_t* qs = a.q + int64_t(b) * a.q_sb + int64_t(h) * a.q_sh + 16 * dq;
      uint16_t* qd = a.pq + (row * a.q_heads + h) * D + 16 * dq;
      *reinterpret_cast<uint4*>(qd) = ld16(qs);
      *reinterpret_cast<uint4*>(qd + 8) = ld16(qs + 8);
      if (dq == 0) a.pnorm[row * a.q_heads + h] = norm;
    }
    if (threadIdx.x == 0) a.plen[row] = live ? int32_t(len) : 0;
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

extern "C" int64_t gse_decode_workspace_bytes(int bs, int max_splits, int q_heads, int head_dim) {
  return int64_t(bs) * max_splits * q_heads * (head_dim + 4) * int64_t(sizeof(float)) + int64_t(bs) * q_heads * 4;
}

namespace {

int check_decode_shape(int q_heads, int kv_heads, int head_dim, int chunk, int max_splits) {
  if (head_dim != D) return gse_fail(GSE_ESHAPE, "decode: head_dim must be 64");
  if (kv_heads < 1 || kv_heads > MAX_KVH || q_heads != GROUP * kv_heads)
    return gse_fail(GSE_ESHAPE, "decode: need q_heads == 8 * kv_heads and 1 <= kv_heads <= 8");
  if (chunk < TILE || chunk % TILE) return gse_fail(GSE_EINVAL, "decode: chunk must be a positive multiple of 32");
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
                          int rows_dtype, float* scores, int64_t scores_stride_g,
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

  float* part = static_cast<float*>(workspace);
  float* norm_ws = part + int64_t(bs) * max_splits * q_heads * PART;
  float* norm = norm_out ? norm_out : norm_ws;

  DecodeArgs a = {};
  a.q = static_cast<const uint16_t*>(q);
  a.q_sb = q_stride_b;
  a.q_sh = q_stride_h;
  a.k = static_cast<const uint16_t*>(k_pool);
  a.v = static_cast<const uint16_t*>(v_pool);
  a.kv_ss = kv_stride_s;
  a.kv_sh = kv_stride_h;
  a.src.indptr = kv_indptr;
  a.src.indices = kv_indices;
  a.sinks = sinks;
  a.sinks_dtype = sinks_dtype;
  a.mode = mode_by_row;
  a.rows = rows;
  a.rows_dtype = rows_dtype;
  a.scores = scores;
  a.scores_sg = scores_stride_g;
  a.part = part;
  a.q_heads = q_heads;
  a.kv_heads = kv_heads;
  a.chunk = chunk;
  a.max_splits = max_splits;
  a.scale2 = sm_scale * kLog2e;

  MergeArgs m = {};
  m.part = part;
  m.indptr = kv_indptr;
  m.sinks = sinks;
  m.sinks_dtype = sinks_dtype;
  m.o = static_cast<uint16_t*>(o);
  m.o_sb = o_stride_b;
  m.o_sh = o_stride_h;
  m.norm_out = norm;
  m.q = a.q;
  m.q_sb = q_stride_b;
  m.q_sh = q_stride_h;
  m.mode = mode_by_row;
  m.rows = rows;
  m.rows_dtype = rows_dtype;
  m.q_heads = q_heads;
  m.chunk = chunk;
  m.max_splits = max_splits;

  int rc;
  if (score_mode == GSE_SCORE_LAG) {
    a.sq = static_cast<const uint16_t*>(pend_q);
    a.sq_sb = int64_t(q_heads) * D;
    a.sq_sh = D;
    a.snorm = pend_norm;
    a.snorm_sb = q_heads;
    a.slen = pend_len;
    a.score_by_row = 1;
    if ((rc = launch_split<true, true, false>(a, indices_dtype, bs, s))) return rc;
    m.pq = static_cast<uint16_t*>(pend_q);
    m.pnorm = pend_norm;
    m.plen = pend_len;
  } else {
    if ((rc = launch_split<true, false, false>(a, indices_dtype, bs, s))) return rc;
  }
  hipLaunchKernelGGL(decode_merge_kernel, dim3(bs), dim3(256), 0, s, m);
  if ((rc = gse_launch_check("decode_merge"))) return rc;
  if (score_mode == GSE_SCORE_EAGER) {
    a.sq = a.q;
    a.sq_sb = q_stride_b;
    a.sq_sh = q_stride_h;
    a.snorm = norm;
    a.snorm_sb = q_heads;
    a.slen = nullptr;
    a.score_by_row = 0;
    if ((rc = launch_split<false, true, false>(a, indices_dtype, bs, s))) return rc;
  }
  return GSE_OK;
}

extern "C" int gse_decode_flush(const void* k_pool, int64_t kv_stride_s, int64_t kv_stride_h,
                                const int32_t* table, int64_t table_stride, const int32_t* req_to_token,
                                int64_t r2t_stride, int64_t r2t_width, const int32_t* frontier, const int32_t* count,
                                const int32_t* mode_by_row, const void* rows, int rows_dtype, int n_rows,
                                float* scores, int64_t scores_stride_g, void* pend_q, float* pend_norm,
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
                                          int64_t scores_stride_g, int bs, int q_heads, int kv_heads,
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
