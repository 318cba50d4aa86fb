// Chunked-prefill score tiles on MFMA (gfx950): exact probabilities with the
// sink in the normaliser, reduced per KV head over its query heads (sum or
// max) and over the chunk's queries, added to each key's slot score.
//
// A workgroup owns one KV head and 64 queries (4 waves x 16). Its MFMA rows
// are (query, head) pairs: row-block rb of a wave holds queries 2*rb and
// 2*rb + 1 with the KV head's 8 query heads each, so no row is padding:
//   S = Q . K^T   [16 rows x 16 keys] per row-block and key-block (16x16x32 bf16)
// Pass 1 streams the visible keys once to get each row's log-sum-exp (with the
// sink); pass 2 streams them again, turns logits into probabilities with that
// normaliser and accumulates column sums, one atomic add per key per workgroup.
#include "common.hpp"
#include "host.hpp"

namespace gse {

namespace pf {
constexpr int D = 64;
constexpr int GROUP = 8;
constexpr int QB = 64;     // queries per workgroup
constexpr int RB = 8;      // row-blocks per wave (16 queries)
constexpr int KT = 64;     // keys per tile (4 key-blocks of 16)
}  // namespace pf

struct PrefillArgs {
  const uint16_t* q;
  int64_t q_st, q_sh;
  int64_t count;
  const uint16_t* k;
  int64_t kv_ss, kv_sh;
  const void* slots;
  int slots_dtype;
  int64_t total, prefix_len;
  const void* sinks;
  int sinks_dtype;
  int mode;
  float* scores;
  int64_t ssg, sss;
  int q_heads, kv_heads;
  float scale2;
  float* norm2;  // [count, q_heads] row normalisers in log2 units (sink included)
};

template <int PASS>
__global__ __launch_bounds__(256) void prefill_kernel(PrefillArgs a) {
  using namespace pf;
  __shared__ float colsum[KT];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const int g = blockIdx.y;
  const int64_t qb0 = int64_t(blockIdx.x) * QB;
  const int64_t i0 = qb0 + 16 * wave;  // this wave's first query
  // Keys visible to any query of the workgroup: CSR columns <= prefix_len + last query.
  const int64_t last_q = (qb0 + QB < a.count ? qb0 + QB : a.count) - 1;
  const int64_t kend = a.prefix_len + last_q + 1 < a.total ? a.prefix_len + last_q + 1 : a.total;

  // A fragments: row col of row-block rb is query i0 + 2*rb + col/8, head g*8 + col%8;
  // lane supplies dims [16*grp, 16*grp + 16) as two 8-dim MFMA halves.
  bf16x8_t qa[RB][2];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int64_t qi = i0 + 2 * rb + col / 8;
    if (qi < a.count) {
      const uint16_t* qp = a.q + qi * a.q_st + int64_t(g * GROUP + col % 8) * a.q_sh + 16 * grp;
      qa[rb][0] = as_bf16x8(*reinterpret_cast<const uint4*>(qp));
      qa[rb][1] = as_bf16x8(*reinterpret_cast<const uint4*>(qp + 8));
    } else {
      qa[rb][0] = bf16x8_t{};
      qa[rb][1] = bf16x8_t{};
    }
  }
  // Output rows of this lane in row-block rb: query i0 + 2*rb + grp/2, heads 4*(grp%2) + r.
  const int hq0 = g * GROUP + 4 * (grp & 1);

  float m[RB][4], l[RB][4], nrm[RB][4];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      m[rb][r] = -INFINITY;
      l[rb][r] = 0.f;
      nrm[rb][r] = 0.f;
    }
  if (PASS == 2) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int64_t qi = i0 + 2 * rb + (grp >> 1);
      if (qi < a.count)
#pragma unroll
        for (int r = 0; r < 4; ++r) nrm[rb][r] = a.norm2[qi * a.q_heads + hq0 + r];
    }
    if (threadIdx.x < KT) colsum[threadIdx.x] = 0.f;
    __syncthreads();
  }
  const bool max_mode = a.mode == 2;

  for (int64_t t0 = 0; t0 < kend; t0 += KT) {
    // B fragments: key t0 + 16*kb + col, dims [16*grp, 16*grp + 16).
    uint4 kf[4][2];
    int64_t slot[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const int64_t key = t0 + 16 * kb + col;
      slot[kb] = key < kend ? load_index_dyn(a.slots, a.slots_dtype, key) : 0;
      const uint16_t* kp = a.k + slot[kb] * a.kv_ss + int64_t(g) * a.kv_sh + 16 * grp;
      kf[kb][0] = *reinterpret_cast<const uint4*>(kp);
      kf[kb][1] = *reinterpret_cast<const uint4*>(kp + 8);
    }
    // Causal mask is needed only where the tile reaches past this wave's first query.
    const bool need_mask = t0 + KT - 1 > a.prefix_len + i0 || t0 + KT > kend;
    float cs[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int64_t qi = i0 + 2 * rb + (grp >> 1);
      const int64_t qpos = a.prefix_len + qi;
      const bool row_dead = qi >= a.count;  // rows past the chunk carry zero queries
      float x[4][4];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
        acc = mfma16x16x32(qa[rb][0], as_bf16x8(kf[kb][0]), acc);
        acc = mfma16x16x32(qa[rb][1], as_bf16x8(kf[kb][1]), acc);
        const int64_t key = t0 + 16 * kb + col;
        const bool dead = row_dead || (need_mask && (key > qpos || key >= kend));
#pragma unroll
        for (int r = 0; r < 4; ++r) x[kb][r] = dead ? -INFINITY : acc[r] * a.scale2;
      }
      if (PASS == 1) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float tm = fmaxf(fmaxf(x[0][r], x[1][r]), fmaxf(x[2][r], x[3][r]));
          const float mn = fmaxf(m[rb][r], tm);
          if (mn != -INFINITY) {
            l[rb][r] = l[rb][r] * fast_exp2(m[rb][r] - mn) + fast_exp2(x[0][r] - mn) + fast_exp2(x[1][r] - mn) +
                       fast_exp2(x[2][r] - mn) + fast_exp2(x[3][r] - mn);
            m[rb][r] = mn;
          }
        }
      } else {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          float red = 0.f;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float p = fast_exp2(x[kb][r] - nrm[rb][r]);
            red = max_mode ? fmaxf(red, p) : red + p;
          }
          // Heads 0-3 (groups 0, 2) with heads 4-7 (groups 1, 3) of the same query.
          red = max_mode ? xor16_max(red) : xor16_sum(red);
          cs[kb] += red;
        }
      }
    }
    if (PASS == 2) {
      // Groups 0/1 hold the even queries' sums, groups 2/3 the odd ones'.
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const float tot = xor32_sum(cs[kb]);
        if (grp == 0 && t0 + 16 * kb + col < kend) atomicAdd(&colsum[16 * kb + col], tot);
      }
      __syncthreads();
      if (threadIdx.x < KT) {
        const int64_t key = t0 + threadIdx.x;
        if (key < kend) {
          const int64_t s = load_index_dyn(a.slots, a.slots_dtype, key);
          unsafeAtomicAdd(&a.scores[int64_t(g) * a.ssg + s * a.sss], colsum[threadIdx.x]);
        }
        colsum[threadIdx.x] = 0.f;
      }
      __syncthreads();
    }
  }

  if (PASS == 1) {
    // Combine each row's (m, l) over the 16 key columns, then fold in the sink.
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float mm = m[rb][r], ll = l[rb][r];
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) {
          const float mo = __shfl_xor(mm, o, kWave), lo = __shfl_xor(ll, o, kWave);
          const float mn = fmaxf(mm, mo);
          ll = (mm == -INFINITY ? 0.f : ll * fast_exp2(mm - mn)) + (mo == -INFINITY ? 0.f : lo * fast_exp2(mo - mn));
          mm = mn;
        }
        const int64_t qi = i0 + 2 * rb + (grp >> 1);
        if (col == 0 && qi < a.count) {
          const float sink2 = load_float_dyn(a.sinks, a.sinks_dtype, hq0 + r) * kLog2e;
          const float mx = fmaxf(mm, sink2);
          a.norm2[qi * a.q_heads + hq0 + r] = mx + __log2f(ll * fast_exp2(mm - mx) + fast_exp2(sink2 - mx));
        }
      }
  }
}

}  // namespace gse

using namespace gse;

extern "C" int64_t gse_prefill_workspace_bytes(int64_t count, int q_heads) {
  return ((count * q_heads * 4 + 255) / 256) * 256;
}

extern "C" int gse_prefill_scores(const void* q, int64_t q_stride_t, int64_t q_stride_h, int64_t count,
                                  const void* k_pool, int64_t kv_stride_s, int64_t kv_stride_h, const void* slots,
                                  int slots_dtype, int64_t total, int64_t prefix_len, const void* sinks,
                                  int sinks_dtype, int mode, float* scores, int64_t scores_stride_g,
                                  int64_t scores_stride_s, int q_heads, int kv_heads, int head_dim, float sm_scale,
                                  void* workspace, int64_t workspace_bytes, gse_stream_t stream) {
  if (head_dim != pf::D || kv_heads < 1 || q_heads != pf::GROUP * kv_heads)
    return gse_fail(GSE_ESHAPE, "prefill: need head_dim 64 and q_heads == 8 * kv_heads");
  if (mode != 1 && mode != 2) return gse_fail(GSE_EINVAL, "prefill: mode must be 1 (sum) or 2 (max)");
  if (count < 0 || prefix_len < 0 || total != prefix_len + count)
    return gse_fail(GSE_EINVAL, "prefill: total must equal prefix_len + count");
  if (count == 0) return GSE_OK;
  if (q_stride_t % 8 || q_stride_h % 8 || kv_stride_s % 8 || kv_stride_h % 8)
    return gse_fail(GSE_EINVAL, "prefill: strides must be multiples of 8 elements");
  if (!q || !k_pool || !slots || !sinks || !scores) return gse_fail(GSE_EINVAL, "prefill: null pointer");
  if (workspace_bytes < gse_prefill_workspace_bytes(count, q_heads))
    return gse_fail(GSE_EWORKSPACE, "prefill: workspace too small");
  PrefillArgs a = {static_cast<const uint16_t*>(q), q_stride_t, q_stride_h, count,
                   static_cast<const uint16_t*>(k_pool), kv_stride_s, kv_stride_h, slots, slots_dtype, total,
                   prefix_len, sinks, sinks_dtype, mode, scores, scores_stride_g, scores_stride_s, q_heads, kv_heads,
                   sm_scale * kLog2e, static_cast<float*>(workspace)};
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(unsigned((count + pf::QB - 1) / pf::QB), unsigned(kv_heads));
  hipLaunchKernelGGL(prefill_kernel<1>, grid, dim3(256), 0, s, a);
  if (int rc = gse_launch_check("prefill pass 1")) return rc;
  hipLaunchKernelGGL(prefill_kernel<2>, grid, dim3(256), 0, s, a);
  return gse_launch_check("prefill pass 2");
}
