// The writer half of the QKV step after the projection: per-head RMSNorm of Q and K (optional), rotate-half RoPE of
// Q and K, Q written out and K / V stored into the paged MHA pool (bf16, or e4m3fn with per-KV-head scales), in one
// pass over the projection's output.
//
// Work: one wave per (token, head) unit, heads ordered [Q 0 .. Hq) [K 0 .. Hkv) [V 0 .. Hkv) as the fused projection
// lays them out. Lane l < d / 2 holds the rotate-half pair (l, l + d / 2), so RoPE needs no exchange and the norm's
// sum of squares is one wave reduction. Every rounding step of the reference's torch path is kept: the norm rounds
// x * rsqrt(mean + eps) to bf16 and multiplies by the bf16 gamma with a bf16 result; RoPE rounds each product and the
// sum to bf16. The sum of squares is fp32 in a wave-reduction order, so with the norm on a value can differ from the
// reference's by one bf16 step where that order changes the sum's last bit; without the norm the path is bit-exact.
#include "sna_device.h"
#include "sna_host.h"

namespace sna {

__device__ __forceinline__ float bf16_round(float x) { return bf16_bits_to_f32(f32_to_bf16_bits(x)); }

template <bool FP8>
__global__ __launch_bounds__(256) void qkv_norm_rope_store_kernel(
    const uint16_t* __restrict__ qkv, int64_t qkv_stride, int64_t n_tokens, int32_t Hq, int32_t Hkv, int32_t D,
    const uint16_t* __restrict__ q_norm, const uint16_t* __restrict__ k_norm, float eps,
    const uint16_t* __restrict__ cosv, const uint16_t* __restrict__ sinv, int64_t rope_stride,
    const int64_t* __restrict__ slots, uint16_t* __restrict__ q_out, uint8_t* __restrict__ kc,
    uint8_t* __restrict__ vc, const float* __restrict__ k_scale, const float* __restrict__ v_scale,
    int64_t num_slots, int32_t P) {
  const int lane = threadIdx.x & 63;
  const int32_t heads = Hq + 2 * Hkv;
  const int64_t units = n_tokens * heads;
  const int32_t half = D / 2;
  const bool live = lane < half;
  for (int64_t u = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); u < units; u += (int64_t)gridDim.x * 4) {
    const int64_t t = u / heads;
    const int32_t head = (int32_t)(u % heads);  // uniform per wave
    const uint16_t* src = qkv + t * qkv_stride + (int64_t)head * D;
    float x0 = live ? bf16_bits_to_f32(src[lane]) : 0.0f;
    float x1 = live ? bf16_bits_to_f32(src[lane + half]) : 0.0f;
    if (head < Hq + Hkv) {
      const bool is_q = head < Hq;
      const uint16_t* gamma = is_q ? q_norm : k_norm;
      if (gamma) {
        // _rms: gamma * (x32 * rsqrt(mean(x32^2) + eps)).to(bf16), rsqrt as 1 / sqrt (both correctly rounded)
        const float ss = wave_sum(x0 * x0 + x1 * x1);
        const float inv = 1.0f / __fsqrt_rn(ss / (float)D + eps);
        if (live) {
          x0 = bf16_round(bf16_bits_to_f32(gamma[lane]) * bf16_round(x0 * inv));
          x1 = bf16_round(bf16_bits_to_f32(gamma[lane + half]) * bf16_round(x1 * inv));
        }
      }
      if (!live) continue;
      // rope(t) = t * c + cat(-t[half:], t[:half]) * s, every product and the sum rounded to bf16
      const uint16_t* cr = cosv + t * rope_stride;
      const uint16_t* sr = sinv + t * rope_stride;
      const float c0 = bf16_bits_to_f32(cr[lane]), c1 = bf16_bits_to_f32(cr[lane + half]);
      const float s0 = bf16_bits_to_f32(sr[lane]), s1 = bf16_bits_to_f32(sr[lane + half]);
      const float y0 = bf16_round(bf16_round(x0 * c0) + bf16_round(-x1 * s0));
      const float y1 = bf16_round(bf16_round(x1 * c1) + bf16_round(x0 * s1));
      if (is_q) {
        uint16_t* dst = q_out + (t * Hq + head) * D;
        dst[lane] = (uint16_t)f32_to_bf16_bits(y0);
        dst[lane + half] = (uint16_t)f32_to_bf16_bits(y1);
        continue;
      }
      x0 = y0;
      x1 = y1;
    }
    if (!live) continue;
    // K (rotated) or V into the pool at the token's slot, as the MHA store writes it
    const bool is_k = head < Hq + Hkv;
    const int32_t h = head - Hq - (is_k ? 0 : Hkv);
    const int64_t slot = redirect_slot(slots[t], num_slots);
    const int64_t dst = (((slot / P) * Hkv + h) * P + slot % P) * D + lane;
    uint8_t* cache = is_k ? kc : vc;
    if constexpr (FP8) {
      const float s = is_k ? k_scale[h] : v_scale[h];
      cache[dst] = (uint8_t)quantize_e4m3fn(f32_to_bf16_bits(x0), s);
      cache[dst + half] = (uint8_t)quantize_e4m3fn(f32_to_bf16_bits(x1), s);
    } else {
      reinterpret_cast<uint16_t*>(cache)[dst] = (uint16_t)f32_to_bf16_bits(x0);
      reinterpret_cast<uint16_t*>(cache)[dst + half] = (uint16_t)f32_to_bf16_bits(x1);
    }
  }
}

}  // namespace sna

using namespace sna;

extern "C" int sna_qkv_norm_rope_store(const void* qkv, int64_t qkv_stride, int64_t n_tokens, int32_t num_q_heads,
                                       int32_t num_kv_heads, int32_t head_dim, const void* q_norm,
                                       const void* k_norm, float eps, const void* cos, const void* sin,
                                       int64_t rope_stride, const int64_t* slots, void* q_out, void* k_cache,
                                       void* v_cache, const float* k_scale, const float* v_scale, int64_t num_blocks,
                                       int32_t page_size, int32_t cache_dtype, void* stream) {
  ApiGuard guard;
  if (n_tokens < 0 || num_q_heads < 1 || num_kv_heads < 1 || head_dim < 2 || head_dim > 128 || head_dim % 2 ||
      page_size < 1 || num_blocks < 1)
    return fail(SNA_ERR_INVALID_ARGUMENT,
                "qkv_norm_rope_store: bad sizes (tokens %lld, heads %d/%d, head_dim %d (even, <= 128), page %d, "
                "blocks %lld)",
                (long long)n_tokens, num_q_heads, num_kv_heads, head_dim, page_size, (long long)num_blocks);
  if (qkv_stride < (int64_t)(num_q_heads + 2 * num_kv_heads) * head_dim || rope_stride < head_dim)
    return fail(SNA_ERR_INVALID_ARGUMENT, "qkv_norm_rope_store: row strides %lld / %lld are shorter than a row",
                (long long)qkv_stride, (long long)rope_stride);
  if ((q_norm == nullptr) != (k_norm == nullptr))
    return fail(SNA_ERR_INVALID_ARGUMENT, "qkv_norm_rope_store: give both QK-norm gammas or neither");
  if (cache_dtype != SNA_DTYPE_BF16 && cache_dtype != SNA_DTYPE_FP8_E4M3FN)
    return fail(SNA_ERR_INVALID_ARGUMENT, "qkv_norm_rope_store: unknown cache dtype %d", cache_dtype);
  const bool fp8 = cache_dtype == SNA_DTYPE_FP8_E4M3FN;
  if (n_tokens == 0) return SNA_OK;
  if (!qkv || !cos || !sin || !slots || !q_out || !k_cache || !v_cache || (fp8 && (!k_scale || !v_scale)))
    return fail(SNA_ERR_INVALID_ARGUMENT, "qkv_norm_rope_store: null pointer");
  if (!(eps >= 0.0f)) return fail(SNA_ERR_INVALID_ARGUMENT, "qkv_norm_rope_store: eps %g", (double)eps);
  const int64_t units = n_tokens * (num_q_heads + 2 * num_kv_heads);
  const unsigned grid = (unsigned)std::min<int64_t>((units + 3) / 4, 65536);
  const int64_t num_slots = num_blocks * page_size;
  hipStream_t s = (hipStream_t)stream;
  if (fp8)
    hipLaunchKernelGGL(qkv_norm_rope_store_kernel<true>, dim3(grid), dim3(256), 0, s, (const uint16_t*)qkv,
                       qkv_stride, n_tokens, num_q_heads, num_kv_heads, head_dim, (const uint16_t*)q_norm,
                       (const uint16_t*)k_norm, eps, (const uint16_t*)cos, (const uint16_t*)sin, rope_stride, slots,
                       (uint16_t*)q_out, (uint8_t*)k_cache, (uint8_t*)v_cache, k_scale, v_scale, num_slots,
                       page_size);
  else
    hipLaunchKernelGGL(qkv_norm_rope_store_kernel<false>, dim3(grid), dim3(256), 0, s, (const uint16_t*)qkv,
                       qkv_stride, n_tokens, num_q_heads, num_kv_heads, head_dim, (const uint16_t*)q_norm,
                       (const uint16_t*)k_norm, eps, (const uint16_t*)cos, (const uint16_t*)sin, rope_stride, slots,
                       (uint16_t*)q_out, (uint8_t*)k_cache, (uint8_t*)v_cache, k_scale, v_scale, num_slots,
                       page_size);
  return check_launch("qkv_norm_rope_store");
}
