// CSR of resident slots for the full-attention layers, and the per-step score reset.
#include "common.hpp"
#include "host.hpp"

namespace gse {

struct FillArgs {
  const int32_t* table;
  int64_t table_stride;
  const int32_t* r2t;
  int64_t r2t_stride;
  const void* rows;
  int rows_dtype;
  const void* lens;
  int lens_dtype;
  const int32_t* frontier;
  const int32_t* count;
  int bs;
  int32_t* indptr;
  void* indices;
};

GSE_DEVICE int64_t fill_size(const FillArgs& a, int i) {
  const int64_t row = load_index_dyn(a.rows, a.rows_dtype, i);
  return load_index_dyn(a.lens, a.lens_dtype, i) - a.frontier[row] + a.count[row];
}

// Grid (bs, segments of FILL_SEG entries): each workgroup finds its entry's CSR offset (the
// sum of the sizes before it, reduced in the workgroup) and copies one segment of the
// entry's list (table part, then tail); workgroups past the entry's list only exit.
constexpr int FILL_SEG = 2048;

template <typename OutT>
__global__ __launch_bounds__(256) void fill_kernel(FillArgs a) {
  __shared__ int64_t red[256];
  const int b = blockIdx.x;
  int64_t part = 0;
  for (int i = threadIdx.x; i < b; i += blockDim.x) part += fill_size(a, i);
  red[threadIdx.x] = part;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  const int64_t start = red[0];
  const int64_t row = load_index_dyn(a.rows, a.rows_dtype, b);
  const int64_t cnt = a.count[row];
  const int64_t fr = a.frontier[row];
  const int64_t total = cnt + load_index_dyn(a.lens, a.lens_dtype, b) - fr;
  if (blockIdx.y == 0 && threadIdx.x == 0) {
    a.indptr[b + 1] = int32_t(start + total);
    if (b == 0) a.indptr[0] = 0;
  }
  const int64_t lo = int64_t(blockIdx.y) * FILL_SEG;
  const int64_t hi = lo + FILL_SEG < total ? lo + FILL_SEG : total;
  OutT* out = static_cast<OutT*>(a.indices) + start;
  const int32_t* trow = a.table + row * a.table_stride;
  const int32_t* rrow = a.r2t + row * a.r2t_stride + fr - cnt;  // entry i >= cnt is rrow[i]
  for (int64_t i = lo + threadIdx.x; i < hi; i += blockDim.x) out[i] = OutT(i < cnt ? trow[i] : rrow[i]);
}

template <typename SlotT>
__global__ void zero_slots_kernel(float* scores, int layers, int64_t layer_stride, int kv_heads, int64_t head_stride,
                                  int64_t slot_stride, const SlotT* slots, int64_t n) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n * layers * kv_heads) return;
  const int64_t s = i % n;
  const int64_t lg = i / n;
  const int64_t g = lg % kv_heads, l = lg / kv_heads;
  scores[l * layer_stride + g * head_stride + int64_t(slots[s]) * slot_stride] = 0.f;
}

}  // namespace gse

using namespace gse;

extern "C" int gse_fill(const int32_t* table, int64_t table_stride, const int32_t* req_to_token, int64_t r2t_stride,
                        const void* rows, int rows_dtype, const void* seq_lens, int lens_dtype,
                        const int32_t* frontier, const int32_t* count, int bs, int64_t max_len,
                        int32_t* kv_indptr, void* kv_indices, int indices_dtype, gse_stream_t stream) {
  if (bs < 0) return gse_fail(GSE_EINVAL, "fill: bs < 0");
  if (bs == 0) return GSE_OK;
  if (!table || !req_to_token || !rows || !seq_lens || !frontier || !count || !kv_indptr || !kv_indices)
    return gse_fail(GSE_EINVAL, "fill: null pointer");
  FillArgs a = {table, table_stride, req_to_token, r2t_stride, rows, rows_dtype, seq_lens, lens_dtype,
                frontier, count, bs, kv_indptr, kv_indices};
  if (max_len < 0) return gse_fail(GSE_EINVAL, "fill: max_len < 0");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<uint32_t>(bs), static_cast<uint32_t>((max_len + FILL_SEG - 1) / FILL_SEG + 1));
  if (indices_dtype == GSE_I64)
    hipLaunchKernelGGL(fill_kernel<int64_t>, grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(fill_kernel<int32_t>, grid, dim3(256), 0, s, a);
  return gse_launch_check("fill");
}

extern "C" int gse_zero_slots(float* scores, int layers, int64_t layer_stride, int kv_heads, int64_t head_stride,
                              int64_t slot_stride, const void* slots, int slots_dtype, int64_t n, gse_stream_t stream) {
  if (n < 0 || layers < 0 || kv_heads < 0) return gse_fail(GSE_EINVAL, "zero_slots: negative size");
  const int64_t total = n * layers * kv_heads;
  if (total == 0) return GSE_OK;
  if (!scores || !slots) return gse_fail(GSE_EINVAL, "zero_slots: null pointer");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(unsigned((total + 255) / 256));
  if (slots_dtype == GSE_I64)
    hipLaunchKernelGGL(zero_slots_kernel<int64_t>, grid, dim3(256), 0, s, scores, layers, layer_stride, kv_heads,
                       head_stride, slot_stride, static_cast<const int64_t*>(slots), n);
  else
    hipLaunchKernelGGL(zero_slots_kernel<int32_t>, grid, dim3(256), 0, s, scores, layers, layer_stride, kv_heads,
                       head_stride, slot_stride, static_cast<const int32_t*>(slots), n);
  return gse_launch_check("zero_slots");
}
