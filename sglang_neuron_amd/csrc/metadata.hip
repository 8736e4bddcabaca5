// Decode metadata on the device: the block table from SGLang's req_to_token map, and a sliding-window layer's
// trimmed table. Both are gathers of 4-byte entries (HBM-bound, one thread per output entry), so a forward's
// metadata never leaves the GPU: no host view of req_to_token, no per-step upload.
//
//   block table (attention/backend.py:114-130): table[b, j] = floor(req_to_token[row_b, j * P] / P) while
//     j * P < seq_len_b, else -1;
//   window trim (model_executor/graph_runner.py:1121-1133): start_b = max(floor((seq_len_b - 1) / P) - nb + 1, 0),
//     trimmed[b, i] = table[b, start_b + i] inside the table's width, else -1; offset_b = start_b * P.

#include "sna_device.h"
#include "sna_host.h"

namespace sna {

__device__ __forceinline__ int64_t floor_div(int64_t x, int64_t d) {  // d > 0
  const int64_t q = x / d;
  return (x % d != 0 && x < 0) ? q - 1 : q;
}

__global__ __launch_bounds__(256) void block_table_kernel(const int32_t* r2t, int64_t r2t_rows, int64_t r2t_width,
                                                          int64_t r2t_stride, const int64_t* rows,
                                                          const int64_t* lens, int32_t B, int32_t P, int32_t width,
                                                          int32_t* table, int32_t* lens32) {
  const int64_t n = (int64_t)B * width;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    const int32_t b = (int32_t)(e / width), j = (int32_t)(e % width);
    const int64_t row = rows[b], len = lens[b], tok = (int64_t)j * P;
    int32_t v = -1;
    if (row >= 0 && row < r2t_rows && tok < len && tok < r2t_width)
      v = (int32_t)floor_div(r2t[row * r2t_stride + tok], P);
    table[e] = v;
    if (lens32 && j == 0) lens32[b] = (int32_t)len;
  }
}

__global__ __launch_bounds__(256) void window_table_kernel(const int32_t* table, int64_t table_stride,
                                                           int32_t table_width, const int64_t* lens, int32_t B,
                                                           int32_t P, int32_t nb, int32_t* trimmed,
                                                           int32_t* offset) {
  const int64_t n = (int64_t)B * nb;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    const int32_t b = (int32_t)(e / nb), i = (int32_t)(e % nb);
    const int64_t start = max(floor_div(lens[b] - 1, P) - nb + 1, (int64_t)0);
    const int64_t col = start + i;
    trimmed[e] = col < table_width ? table[(int64_t)b * table_stride + col] : -1;
    if (i == 0) offset[b] = (int32_t)(start * P);
  }
}

static unsigned grid_for(int64_t n) { return (unsigned)std::min<int64_t>((n + 255) / 256, 8192); }

}  // namespace sna

using namespace sna;

extern "C" {

int sna_block_table(const int32_t* req_to_token, int64_t r2t_rows, int64_t r2t_width, int64_t r2t_stride,
                    const int64_t* req_pool_indices, const int64_t* seq_lens, int32_t B, int32_t page_size,
                    int32_t width, int32_t* table, int32_t* seq_lens_i32, void* stream) {
  ApiGuard guard;
  if (B < 0 || width < 1 || page_size < 1 || r2t_rows < 0 || r2t_width < 0 || r2t_stride < r2t_width)
    return fail(SNA_ERR_INVALID_ARGUMENT,
                "block_table: bad sizes (B %d, width %d, page %d, req_to_token %lld x %lld, stride %lld)", B, width,
                page_size, (long long)r2t_rows, (long long)r2t_width, (long long)r2t_stride);
  if (B == 0) return SNA_OK;
  if (!req_to_token || !req_pool_indices || !seq_lens || !table)
    return fail(SNA_ERR_INVALID_ARGUMENT, "block_table: null pointer");
  hipLaunchKernelGGL(block_table_kernel, dim3(grid_for((int64_t)B * width)), dim3(256), 0, (hipStream_t)stream,
                     req_to_token, r2t_rows, r2t_width, r2t_stride, req_pool_indices, seq_lens, B, page_size, width, table,
                     seq_lens_i32);
  return check_launch("block_table");
}

int sna_window_table(const int32_t* table, int64_t table_stride, int32_t table_width, const int64_t* seq_lens,
                     int32_t B, int32_t page_size, int32_t n_blocks, int32_t* trimmed, int32_t* pos_offset,
                     void* stream) {
  ApiGuard guard;
  if (B < 0 || table_width < 1 || table_stride < table_width || page_size < 1 || n_blocks < 1)
    return fail(SNA_ERR_INVALID_ARGUMENT, "window_table: bad sizes (B %d, table %d wide, stride %lld, page %d, %d blocks)",
                B, table_width, (long long)table_stride, page_size, n_blocks);
  if (B == 0) return SNA_OK;
  if (!table || !seq_lens || !trimmed || !pos_offset) return fail(SNA_ERR_INVALID_ARGUMENT, "window_table: null pointer");
  hipLaunchKernelGGL(window_table_kernel, dim3(grid_for((int64_t)B * n_blocks)), dim3(256), 0, (hipStream_t)stream,
                     table, table_stride, table_width, seq_lens, B, page_size, n_blocks, trimmed, pos_offset);
  return check_launch("window_table");
}

}  // extern "C"
