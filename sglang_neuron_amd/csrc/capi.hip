// C ABI plumbing: version, error state, split-K planning and the LSE merge of partial results.
#include <algorithm>
#include <cmath>

#include "sna_device.h"
#include "sna_host.h"

namespace sna {

char* error_buffer() {
  static thread_local char buf[kErrorBufferBytes];
  return buf;
}

namespace {

int32_t host_splits(int32_t seq_len, int32_t window, int32_t tile, int32_t split_tiles) {
  if (seq_len <= 1) return 0;
  int32_t hi = seq_len - 1;
  int32_t lo = (window > 0 && seq_len - window > 0) ? seq_len - window : 0;
  if (hi <= lo) return 0;
  int32_t t0 = lo / tile, t1 = (hi + tile - 1) / tile;
  return (t1 - t0 + split_tiles - 1) / split_tiles;
}

int32_t host_tiles(int32_t seq_len, int32_t window, int32_t tile) { return host_splits(seq_len, window, tile, 1); }

}  // namespace

// ---- LSE merge of partials (decode-context-parallel style) ----
__global__ __launch_bounds__(256) void lse_combine_kernel(const float* __restrict__ o_parts,
                                                          const float* __restrict__ lse_parts, int32_t n_parts,
                                                          int64_t n_rows, int32_t dim, uint16_t* __restrict__ out,
                                                          float* __restrict__ lse_out) {
  const int64_t row = blockIdx.x;
  float m = -INFINITY;
  for (int32_t i = 0; i < n_parts; ++i) m = fmaxf(m, lse_parts[(int64_t)i * n_rows + row]);
  float den = 0.0f;
  for (int32_t i = 0; i < n_parts; ++i) {
    const float l = lse_parts[(int64_t)i * n_rows + row];
    den += (m == -INFINITY) ? 0.0f : expf(l - m);
  }
  const float lse = (m == -INFINITY || den == 0.0f) ? -INFINITY : m + logf(den);
  for (int32_t d = threadIdx.x; d < dim; d += blockDim.x) {
    float acc = 0.0f;
    if (lse != -INFINITY) {
      for (int32_t i = 0; i < n_parts; ++i) {
        const float l = lse_parts[(int64_t)i * n_rows + row];
        if (l == -INFINITY) continue;
        acc += expf(l - lse) * o_parts[((int64_t)i * n_rows + row) * dim + d];
      }
    }
    out[row * dim + d] = (uint16_t)f32_to_bf16_bits(acc);
  }
  if (lse_out && threadIdx.x == 0) lse_out[row] = lse;
}

}  // namespace sna

using namespace sna;

extern "C" {

int sna_version(void) { return 100; }

const char* sna_last_error(void) { return error_buffer(); }

int sna_plan_decode(int32_t kind, const int32_t* host_seq_lens, int32_t B, int32_t max_seq_len, int32_t window,
                    int32_t n_keys_per_row, int32_t ctas_per_item, int32_t num_cus, sna_split_plan* plan) {
  ApiGuard guard;
  if (!plan) return fail(SNA_ERR_INVALID_ARGUMENT, "plan_decode: null plan");
  if (kind < 0 || kind > 2) return fail(SNA_ERR_INVALID_ARGUMENT, "plan_decode: unknown kind %d", kind);
  if (B < 0 || ctas_per_item < 1 || window < 0)
    return fail(SNA_ERR_INVALID_ARGUMENT, "plan_decode: bad arguments (B %d, ctas_per_item %d, window %d)", B,
                ctas_per_item, window);
  if (kind == 2 && n_keys_per_row < 0)
    return fail(SNA_ERR_INVALID_ARGUMENT, "plan_decode: negative index count %d", n_keys_per_row);
  if (kind != 2 && !host_seq_lens && max_seq_len < 0)
    return fail(SNA_ERR_INVALID_ARGUMENT, "plan_decode: need host seq_lens or max_seq_len >= 0");
  const int32_t tile = kind == 0 ? 32 : 16;
  const int32_t waves = 4;
  const int32_t cus = num_cus > 0 ? num_cus : 256;
  // Resident workgroups the launch aims for: GQA runs several 4-wave workgroups per CU; the MLA kernels hold
  // one per CU (their register budget), and the ragged tail is cut by aiming slightly under a full wave of CUs.
  const int64_t target = kind == 0 ? (int64_t)cus * 8 : (int64_t)cus;
  auto len_of = [&](int32_t b) -> int32_t {
    if (kind == 2) return n_keys_per_row + 1;  // the index list as "prior keys" + the own row
    return host_seq_lens ? host_seq_lens[b] : max_seq_len;
  };
  const int32_t win = kind == 2 ? 0 : window;
  int64_t total_tiles = 0;
  int32_t max_tiles = 0;
  for (int32_t b = 0; b < B; ++b) {
    int32_t t = host_tiles(len_of(b), win, tile);
    total_tiles += t;
    max_tiles = std::max(max_tiles, t);
  }
  const int64_t items_target = std::max<int64_t>(1, target / ctas_per_item);
  int32_t split_tiles = (int32_t)std::max<int64_t>(waves, (total_tiles + items_target - 1) / items_target);
  if (kind != 0) {
    // MLA: grow the split until the item count fits the resident target, so no workgroup waits for a second round
    while (true) {
      int64_t n = 0;
      for (int32_t b = 0; b < B; ++b) n += host_splits(len_of(b), win, tile, split_tiles);
      if (n * ctas_per_item <= target || split_tiles >= std::max(max_tiles, waves)) break;
      split_tiles += waves;
    }
  }
  int64_t n_work = 0;
  for (int32_t b = 0; b < B; ++b) n_work += host_splits(len_of(b), win, tile, split_tiles);
  if (n_work > INT32_MAX / 2) return fail(SNA_ERR_INVALID_ARGUMENT, "plan_decode: too many splits");
  plan->split_tiles = split_tiles;
  plan->n_work = (int32_t)n_work;
  plan->tile = tile;
  plan->target_ctas = (int32_t)target;
  return SNA_OK;
}

int64_t sna_decode_workspace_bytes(const sna_split_plan* plan, int32_t num_q_heads, int32_t head_dim_v) {
  if (!plan || num_q_heads < 1 || head_dim_v < 1) return 0;
  return (int64_t)std::max(plan->n_work, 1) * num_q_heads * ((int64_t)head_dim_v + 2) * (int64_t)sizeof(float);
}

int sna_lse_combine(const float* o_parts, const float* lse_parts, int32_t n_parts, int64_t n_rows, int32_t dim,
                    void* out, float* lse_out, void* stream) {
  ApiGuard guard;
  if (n_parts < 1 || n_rows < 0 || dim < 1)
    return fail(SNA_ERR_INVALID_ARGUMENT, "lse_combine: bad sizes (parts %d, rows %lld, dim %d)", n_parts,
                (long long)n_rows, dim);
  if (n_rows == 0) return SNA_OK;
  if (!o_parts || !lse_parts || !out) return fail(SNA_ERR_INVALID_ARGUMENT, "lse_combine: null pointer");
  if (n_rows > INT32_MAX) return fail(SNA_ERR_INVALID_ARGUMENT, "lse_combine: too many rows");
  hipLaunchKernelGGL(lse_combine_kernel, dim3((unsigned)n_rows), dim3(256), 0, (hipStream_t)stream, o_parts,
                     lse_parts, n_parts, n_rows, dim, (uint16_t*)out, lse_out);
  return check_launch("lse_combine");
}

}  // extern "C"
