// Queued decode scores, folded into the score table (gfx950).
//
// The fused decode kernel does attention only; its merge appends each decode
// step's query (all heads), final normaliser (sink included) and slot-list
// length to a per-(layer, row) queue. This pass adds the queued queries' H2O
// scores to every key they saw, the reference's per-step update (R:189-200)
// applied for a batch of steps at once:
//   scores[l, g, slot(c)] += sum_i [c < lim_i] (sum | max)_{h in g} exp(q_ih . k_cg * scale - norm_ih)
// where slot(c) = table[row, c] for c < count[row], else req_to_token[row, frontier[row] + c - count[row]]
// (the list of `fill`, R:136-152); every queued list is a prefix of the current one
// because lists only grow between boundaries, and boundaries flush first.
//
// A workgroup owns one (layer, row, KV head, chunk of keys); its 4 waves take
// 64-key tiles. The queued queries of the KV head sit in LDS; per tile a wave
// keeps K in registers and runs, per pair of queries, D = [Q_i; Q_i+1] . K^T
// ([16 (query, head) rows x 16 keys] per sub-tile, v_mfma_f32_16x16x32_bf16), so a
// lane holds 4 heads of one query for one key: the head reduction is in-lane plus
// one lane swap, and the query sum accumulates in registers. Each key's total is
// added with one atomic per (key, head) at the end: the pass reads K once per
// queue instead of once per step and writes scores once per queue.
#include "common.hpp"
#include "host.hpp"

namespace gse {
namespace fl {
constexpr int D = 64;
constexpr int GROUP = 8;
constexpr int WAVES = 4;
constexpr int TILE = 64;
constexpr int TILES_PER_WAVE = 4;
constexpr int CHUNK = WAVES * TILES_PER_WAVE * TILE;  // keys per workgroup
constexpr int MAX_QUEUE = 64;
constexpr int QROW = D + 8;  // padded bf16 row of a queued (query, head) in LDS
}  // namespace fl

struct FlushArgs {
  void* const* k_pools;  // [layers] device pointers to bf16 [slots, kv_heads, D]
  int64_t kv_ss, kv_sh;
  float* scores;
  int64_t ssl, ssg, sss;
  const int32_t* table;
  int64_t table_stride;
  const int32_t* r2t;
  int64_t r2t_stride;
  const int32_t* frontier;
  const int32_t* count;
  const int32_t* mode;
  const void* rows;
  int rows_dtype;
  // Queues, per layer: q [rows_total, cap, q_heads, D] bf16, norm [rows_total, cap, q_heads],
  // lim [rows_total, cap], n [rows_total].
  const uint16_t* pq;
  const float* pnorm;
  const int32_t* plim;
  int32_t* pcount;
  int rows_total, cap;
  int layers, q_heads, kv_heads;
  float scale2;  // sm_scale * log2(e)
};

// Grid (key chunks, n_rows, layers * kv_heads), 256 threads.
__global__ __launch_bounds__(256) void score_flush_kernel(FlushArgs a) {
  using namespace fl;
  __shared__ __attribute__((aligned(16))) uint16_t qs[MAX_QUEUE * GROUP * QROW];
  __shared__ __attribute__((aligned(16))) float ns[MAX_QUEUE * GROUP];
  __shared__ int lims[MAX_QUEUE];

  const int lg = blockIdx.z;
  const int l = lg / a.kv_heads, g = lg % a.kv_heads;
  const int64_t row = load_index_dyn(a.rows, a.rows_dtype, blockIdx.y);
  const int md = a.mode[row];
  if (md != 1 && md != 2) return;
  const int64_t qbase = int64_t(l) * a.rows_total + row;  // (layer, row) queue index
  int m = a.pcount[qbase];
  m = m < a.cap ? m : a.cap;
  if (m <= 0) return;
  const bool max_mode = md == 2;

  // Queued lengths: the workgroup's keys are [c0, min(c0 + CHUNK, max lim)).
  if (threadIdx.x < m) lims[threadIdx.x] = a.plim[qbase * a.cap + threadIdx.x];
  __syncthreads();
  int maxlim = 0;
  for (int i = 0; i < m; ++i) maxlim = lims[i] > maxlim ? lims[i] : maxlim;
  const int c0 = blockIdx.x * CHUNK;
  if (c0 >= maxlim) return;

  // The KV head's queued (query, head) rows and their normalisers (log2 units) into LDS.
  const uint16_t* qsrc = a.pq + (qbase * a.cap) * a.q_heads * D;
  for (int t = threadIdx.x; t < m * GROUP * (D / 8); t += blockDim.x) {
    const int rowi = t / (D / 8), piece = t % (D / 8);  // rowi = query * 8 + head
    const int qi = rowi / GROUP, h = rowi % GROUP;
    *reinterpret_cast<uint4*>(qs + rowi * QROW + 8 * piece) =
        *reinterpret_cast<const uint4*>(qsrc + (int64_t(qi) * a.q_heads + g * GROUP + h) * D + 8 * piece);
  }
  for (int t = threadIdx.x; t < m * GROUP; t += blockDim.x) {
    const int qi = t / GROUP, h = t % GROUP;
    ns[t] = a.pnorm[(qbase * a.cap + qi) * a.q_heads + g * GROUP + h] * kLog2e;
  }
  // Odd queue lengths: the missing query of the last pair carries no mass.
  if (m & 1) {
    for (int t = threadIdx.x; t < GROUP; t += blockDim.x) ns[m * GROUP + t] = INFINITY;
    for (int t = threadIdx.x; t < GROUP * (D / 8); t += blockDim.x)
      *reinterpret_cast<uint4*>(qs + (m * GROUP + t / (D / 8)) * QROW + 8 * (t % (D / 8))) = uint4{0, 0, 0, 0};
    if (threadIdx.x == 0) lims[m] = 0;
  }
  __syncthreads();

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const int64_t cnt = a.count[row], fr = a.frontier[row];
  const auto kp = as_global(static_cast<const uint16_t*>(a.k_pools[l])) + int64_t(g) * a.kv_sh + 8 * grp;
  float* srow = a.scores + int64_t(l) * a.ssl + int64_t(g) * a.ssg;
  const int npairs = (m + 1) >> 1;

  for (int ti = 0; ti < TILES_PER_WAVE; ++ti) {
    const int tb = c0 + (ti * WAVES + wave) * TILE;
    if (tb >= maxlim) break;
    // Slots and K fragments of keys tb + 16*st + col (lanes past the list read slot 0).
    int32_t slot[4];
    uint4 kf[4][2];
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int c = tb + 16 * st + col;
      const int cc = c < maxlim ? c : maxlim - 1;
      const int32_t s = cc < cnt ? a.table[row * a.table_stride + cc] : a.r2t[row * a.r2t_stride + fr + cc - cnt];
      slot[st] = c < maxlim ? s : 0;
      const auto p = kp + uint64_t(uint32_t(slot[st])) * uint64_t(a.kv_ss);
      kf[st][0] = gload16(p);
      kf[st][1] = gload16(p + 32);
    }
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int pr = 0; pr < npairs; ++pr) {
      // A rows: (query 2*pr + col/8, head col%8); this lane's D rows: query 2*pr + grp/2,
      // heads 4*(grp%2) + r.
      const uint16_t* qrow = qs + ((2 * pr) * GROUP + col) * QROW + 8 * grp;
      const bf16x8_t qa0 = as_bf16x8(*reinterpret_cast<const uint4*>(qrow));
      const bf16x8_t qa1 = as_bf16x8(*reinterpret_cast<const uint4*>(qrow + 32));
      const int qi = 2 * pr + (grp >> 1);
      const f32x4_t nrm = *reinterpret_cast<const f32x4_t*>(ns + qi * GROUP + 4 * (grp & 1));
      const int lim = lims[qi];
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        f32x4_t d = {0.f, 0.f, 0.f, 0.f};
        d = mfma16x16x32(qa0, as_bf16x8(kf[st][0]), d);
        d = mfma16x16x32(qa1, as_bf16x8(kf[st][1]), d);
        const bool live = tb + 16 * st + col < lim;
        float red;
        if (max_mode) {
          red = fmaxf(fmaxf(fast_exp2(fmaf(d[0], a.scale2, -nrm[0])), fast_exp2(fmaf(d[1], a.scale2, -nrm[1]))),
                      fmaxf(fast_exp2(fmaf(d[2], a.scale2, -nrm[2])), fast_exp2(fmaf(d[3], a.scale2, -nrm[3]))));
          red = xor16_max(live ? red : 0.f);
        } else {
          red = (fast_exp2(fmaf(d[0], a.scale2, -nrm[0])) + fast_exp2(fmaf(d[1], a.scale2, -nrm[1]))) +
                (fast_exp2(fmaf(d[2], a.scale2, -nrm[2])) + fast_exp2(fmaf(d[3], a.scale2, -nrm[3])));
          red = xor16_sum(live ? red : 0.f);
        }
        acc[st] += red;
      }
    }
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      // Lanes of groups 0/1 hold even queries' sums, 2/3 odd ones'.
      const float tot = xor32_sum(acc[st]);
      const int c = tb + 16 * st + col;
      if (grp == 0 && c < maxlim) unsafeAtomicAdd(srow + uint64_t(uint32_t(slot[st])) * a.sss, tot);
    }
  }
}

// The queues of the flushed (layer, row) pairs are empty afterwards; a count above the
// capacity (steps the decode merge could not queue) sets *overflow.
__global__ void flush_clear_kernel(const void* rows, int rows_dtype, int n_rows, int layers, int rows_total, int cap,
                                   int32_t* pcount, int32_t* overflow) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_rows * layers) return;
  const int l = i / n_rows;
  int32_t* c = pcount + int64_t(l) * rows_total + load_index_dyn(rows, rows_dtype, i % n_rows);
  if (overflow && *c > cap) *overflow = 1;
  *c = 0;
}

}  // namespace gse

using namespace gse;

extern "C" int gse_score_flush(void* const* k_pools, int layers, int64_t kv_stride_s, int64_t kv_stride_h,
                               float* scores, int64_t scores_stride_l, int64_t scores_stride_g,
                               int64_t scores_stride_s, const int32_t* table, int64_t table_stride,
                               const int32_t* req_to_token, int64_t r2t_stride, const int32_t* frontier,
                               const int32_t* count, const int32_t* mode_by_row, const void* rows, int rows_dtype,
                               int n_rows, int64_t max_len, const void* pend_q, const float* pend_norm,
                               const int32_t* pend_lim, int32_t* pend_count, int rows_total, int queue_cap,
                               int q_heads, int kv_heads, int head_dim, float sm_scale, int32_t* overflow,
                               gse_stream_t stream) {
  using namespace fl;
  if (head_dim != D || kv_heads < 1 || kv_heads > 8 || q_heads != GROUP * kv_heads)
    return gse_fail(GSE_ESHAPE, "score_flush: need head_dim 64 and q_heads == 8 * kv_heads <= 64");
  if (queue_cap < 1 || queue_cap > MAX_QUEUE) return gse_fail(GSE_EINVAL, "score_flush: queue_cap must be 1..64");
  if (n_rows < 0 || layers < 0 || max_len < 0 || rows_total < 0) return gse_fail(GSE_EINVAL, "score_flush: bad sizes");
  if (n_rows == 0 || layers == 0) return GSE_OK;
  if (kv_stride_s % 8 || kv_stride_h % 8) return gse_fail(GSE_EINVAL, "score_flush: K strides must be multiples of 8");
  if (!k_pools || !scores || !table || !req_to_token || !frontier || !count || !mode_by_row || !rows || !pend_q ||
      !pend_norm || !pend_lim || !pend_count)
    return gse_fail(GSE_EINVAL, "score_flush: null pointer");
  if (max_len >= (int64_t(1) << 31)) return gse_fail(GSE_EINVAL, "score_flush: max_len too large");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  FlushArgs f = {k_pools, kv_stride_s, kv_stride_h, scores, scores_stride_l, scores_stride_g, scores_stride_s,
                 table, table_stride, req_to_token, r2t_stride, frontier, count, mode_by_row, rows, rows_dtype,
                 static_cast<const uint16_t*>(pend_q), pend_norm, pend_lim, pend_count, rows_total, queue_cap,
                 layers, q_heads, kv_heads, sm_scale * kLog2e};
  const unsigned chunks = unsigned((max_len + CHUNK - 1) / CHUNK);
  if (chunks) {
    hipLaunchKernelGGL(score_flush_kernel, dim3(chunks, unsigned(n_rows), unsigned(layers * kv_heads)), dim3(256), 0,
                       s, f);
    if (int rc = gse_launch_check("score_flush")) return rc;
  }
  const int total = n_rows * layers;
  hipLaunchKernelGGL(flush_clear_kernel, dim3((total + 255) / 256), dim3(256), 0, s, rows, rows_dtype, n_rows, layers,
                     rows_total, queue_cap, pend_count, overflow);
  return gse_launch_check("score_flush clear");
}
