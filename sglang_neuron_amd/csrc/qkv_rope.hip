// The writer half of the QKV step after the projection: per-head RMSNorm of Q and K (optional), rotate-half RoPE of
// Q and K, Q written out and K / V stored into the paged MHA pool (bf16, or e4m3fn with per-KV-head scales), in one
// pass over the projection's output.
//
// Heads are ordered [Q 0 .. Hq) [K 0 .. Hkv) [V 0 .. Hkv) as the fused projection lays them out. Every rounding step
// of the reference's torch path is kept: the norm rounds x * rsqrt(mean + eps) to bf16 and multiplies by the bf16 gamma with a bf16 result; RoPE rounds each product and the
// sum to bf16. The sum of squares is fp32 in a wave-reduction order, so with the norm on a value can differ from the
// reference's by one bf16 step where that order changes the sum's last bit; without the norm the path is bit-exact.
#include "sna_device.h"
#include "sna_host.h"

namespace sna {

// x rounded to bf16 (nearest even) and back, by the hardware conversion (v_cvt_pk_bf16_f32). It equals
// f32_to_bf16_bits for every non-NaN input; a NaN stays a NaN, and the final conversion of each output writes the
// canonical NaN, as torch does.
__device__ __forceinline__ float bf16_round(float x) { return (float)(__bf16)x; }

// Two floats that are already bf16 values, packed (lo in the low half) by one byte permute.
__device__ __forceinline__ uint32_t pack_exact(float lo, float hi) {
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// The value of the lane `half` lanes away inside the head's lane group (lane ^ half). A 16-lane group (D = 128) is one
// DPP row, where a rotation by 8 is that exchange; other widths go through the LDS crossbar.
template <int HALF>
__device__ __forceinline__ uint32_t partner(uint32_t v) {
  if constexpr (HALF == 8) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xf, 0xf, false);  // row_ror:8
  else return (uint32_t)__shfl_xor((int)v, HALF, 64);
}

// The sum over the head's lane group, in every lane of it, folded in halves: lane i adds the lane HALF away, then
// HALF / 2, ..., 1 (every lane ends with the same bits, addition being commutative). DPP row rotations for a
// 16-lane group (rotations by 8, 4, 2, 1 pair the same lanes there), xor shuffles else.
template <int HALF>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (HALF == 8) {
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xf, 0xf, false));  // row_ror:8
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x124, 0xf, 0xf, false));  // row_ror:4
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x122, 0xf, 0xf, false));  // row_ror:2
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x121, 0xf, 0xf, false));  // row_ror:1
    return v;
  } else {
#pragma unroll
    for (int off = HALF; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
  }
}

// Two floats rounded to bf16 (nearest even) and packed by one conversion, each NaN written as the canonical 0x7FC0
// (f32_to_bf16_bits' and torch's NaN).
__device__ __forceinline__ uint32_t round_pack(float lo, float hi) {
  const bf16x2_t v = __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t);
  uint32_t r = __builtin_bit_cast(uint32_t, v);
  if (lo != lo) r = (r & 0xffff0000u) | 0x7fc0u;
  if (hi != hi) r = (r & 0x0000ffffu) | 0x7fc00000u;
  return r;
}

// Lane layout: a head row of D bf16 is D / 8 lanes of 16 bytes (LPH lanes per head, 64 / LPH heads per wave), so
// every load and store is a 16-byte vector access. Lane j of a head holds elements 8 j .. 8 j + 7; its rotate-half
// partner (the lane LPH / 2 away) holds the elements D / 2 further on, fetched by one xor shuffle per dword. A unit is
// (token, a wave's worth of consecutive heads); a head's type (Q, K, V) is fixed per LPH-lane group.
template <bool FP8, int D>
__global__ __launch_bounds__(256) void qkv_norm_rope_store_kernel(
    const uint16_t* __restrict__ qkv, int64_t qkv_stride, int64_t n_tokens, int32_t Hq, int32_t Hkv,
    const uint16_t* __restrict__ q_norm, const uint16_t* __restrict__ k_norm, float eps,
    const uint16_t* __restrict__ cosv, const uint16_t* __restrict__ sinv, int64_t rope_stride,
    const int64_t* __restrict__ slots, uint16_t* __restrict__ q_out, uint8_t* __restrict__ kc,
    uint8_t* __restrict__ vc, const float* __restrict__ k_scale, const float* __restrict__ v_scale,
    int64_t num_slots, int32_t P) {
  constexpr int LPH = D / 8, HPW = 64 / LPH, HALF = LPH / 2;
  const int lane = threadIdx.x & 63, sub = lane % LPH;
  const int32_t heads = Hq + 2 * Hkv;
  const int32_t groups = (heads + HPW - 1) / HPW;
  const int64_t units = n_tokens * groups;
  const bool first = sub < HALF;
  // U units per wave per pass: the loads of all U are issued before any is computed
  constexpr int U = 1;
  auto process = [&](int64_t u, const uint4& w, const uint4& cw, const uint4& sw) {
    const int64_t t = u / groups;
    const int32_t head = (int32_t)(u % groups) * HPW + lane / LPH;
    const bool live = u < units && head < heads;
    const bool is_q = head < Hq, is_k = !is_q && head < Hq + Hkv;
    float x[8];
    {
      const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = bf16_bits_to_f32((ww[e >> 1] >> (16 * (e & 1))) & 0xffffu);
    }
    if (q_norm) {  // uniform: both gammas or neither
      // _rms: gamma * (x32 * rsqrt(mean(x32^2) + eps)).to(bf16), rsqrt as 1 / sqrt (both correctly rounded). The
      // sum of squares: each square rounded (pow(2)), a lane's 8 summed in sequence, then the head's LPH lane sums
      // folded in halves (group_sum; every lane takes part in the shuffles)
      float ss = 0.0f;
      {
#pragma clang fp contract(off)
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = ss + x[e] * x[e];
      }
      ss = group_sum<HALF>(ss);
      if (live && (is_q || is_k)) {
        const float inv = 1.0f / sqrtf(ss / (float)D + eps);  // sqrtf: correctly rounded (__fsqrt_rn is the native one)
        const uint4 gw = ld16((is_q ? q_norm : k_norm) + 8 * sub);
        const uint32_t gg[4] = {gw.x, gw.y, gw.z, gw.w};
#pragma unroll
        for (int e = 0; e < 8; ++e)
          x[e] = bf16_round(bf16_bits_to_f32((gg[e >> 1] >> (16 * (e & 1))) & 0xffffu) * bf16_round(x[e] * inv));
      }
    }
    // the partner's elements (every lane takes part in the shuffles)
    uint32_t pw[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      pw[e] = partner<HALF>(pack_exact(x[2 * e], x[2 * e + 1]));
    if (!live) return;
    uint32_t ob[4];
    if (is_q || is_k) {
      // rope(t) = t * c + cat(-t[D/2:], t[:D/2]) * s, every product and the sum rounded to bf16 (the sums by the
      // packing conversion)
      const uint32_t cc[4] = {cw.x, cw.y, cw.z, cw.w}, sc[4] = {sw.x, sw.y, sw.z, sw.w};
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        float y[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int e = 2 * e2 + i;
          const float c = bf16_bits_to_f32((cc[e2] >> (16 * i)) & 0xffffu);
          const float sn = bf16_bits_to_f32((sc[e2] >> (16 * i)) & 0xffffu);
          const float p = bf16_bits_to_f32((pw[e2] >> (16 * i)) & 0xffffu);
          y[i] = bf16_round(x[e] * c) + bf16_round((first ? -p : p) * sn);
        }
        ob[e2] = round_pack(y[0], y[1]);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) ob[e] = pack_exact(x[2 * e], x[2 * e + 1]);
    }
    if (is_q) {
      *reinterpret_cast<uint4*>(q_out + (t * Hq + head) * D + 8 * sub) = make_uint4(ob[0], ob[1], ob[2], ob[3]);
      return;
    }
    // K (rotated) or V into the pool at the token's slot, as the MHA store writes it
    const int32_t h = head - Hq - (is_k ? 0 : Hkv);
    const int64_t slot = redirect_slot(slots[t], num_slots);
    const int64_t dst = (((slot / P) * Hkv + h) * P + slot % P) * D + 8 * sub;
    uint8_t* cache = is_k ? kc : vc;
    if constexpr (FP8) {
      const float scl = is_k ? k_scale[h] : v_scale[h];
      uint32_t q8[2] = {0, 0};
      if (rcp_scale_ok(scl)) {
        const float rs = 1.0f / scl;
#pragma unroll
        for (int e = 0; e < 8; ++e)
          q8[e >> 2] |= quantize_e4m3fn_rcp((ob[e >> 1] >> (16 * (e & 1))) & 0xffffu, scl, rs) << (8 * (e & 3));
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          q8[e >> 2] |= quantize_e4m3fn((ob[e >> 1] >> (16 * (e & 1))) & 0xffffu, scl) << (8 * (e & 3));
      }
      *reinterpret_cast<uint2*>(cache + dst) = make_uint2(q8[0], q8[1]);
    } else {
      *reinterpret_cast<uint4*>(cache + 2 * dst) = make_uint4(ob[0], ob[1], ob[2], ob[3]);
    }
  };
  const int64_t stride = (int64_t)gridDim.x * 4 * U;
  for (int64_t base = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * U; base < units; base += stride) {
    uint4 w[U], cw[U], sw[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int64_t u = base + k;
      const int64_t t = u / groups;
      const int32_t head = (int32_t)(u % groups) * HPW + lane / LPH;
      const bool live = u < units && head < heads;
      w[k] = live ? ld16(qkv + t * qkv_stride + (int64_t)head * D + 8 * sub) : make_uint4(0, 0, 0, 0);
      cw[k] = sw[k] = make_uint4(0, 0, 0, 0);
      if (live && head < Hq + Hkv) {
        cw[k] = ld16(cosv + t * rope_stride + 8 * sub);
        sw[k] = ld16(sinv + t * rope_stride + 8 * sub);
      }
    }
#pragma unroll
    for (int k = 0; k < U; ++k) process(base + k, w[k], cw[k], sw[k]);
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
  if (n_tokens < 0 || num_q_heads < 1 || num_kv_heads < 1 || page_size < 1 || num_blocks < 1)
    return fail(SNA_ERR_INVALID_ARGUMENT,
                "qkv_norm_rope_store: bad sizes (tokens %lld, heads %d/%d, head_dim %d, page %d, blocks %lld)",
                (long long)n_tokens, num_q_heads, num_kv_heads, head_dim, page_size, (long long)num_blocks);
  if (head_dim != 64 && head_dim != 128)
    return fail(SNA_ERR_UNSUPPORTED, "qkv_norm_rope_store: head_dim %d (64 or 128 are built)", head_dim);
  if (qkv_stride < (int64_t)(num_q_heads + 2 * num_kv_heads) * head_dim || rope_stride < head_dim)
    return fail(SNA_ERR_INVALID_ARGUMENT, "qkv_norm_rope_store: row strides %lld / %lld are shorter than a row",
                (long long)qkv_stride, (long long)rope_stride);
  if ((q_norm == nullptr) != (k_norm == nullptr))
    return fail(SNA_ERR_INVALID_ARGUMENT, "qkv_norm_rope_store: give both QK-norm gammas or neither");
  if (cache_dtype == SNA_DTYPE_FP8_E4M3FN_MUL)
    return fail(SNA_ERR_UNSUPPORTED, "qkv_norm_rope_store: the writer divides by dequantization scales; for a pool of "
                "GPT-OSS multipliers m pass SNA_DTYPE_FP8_E4M3FN with the scales bf16(1 / m), as the reference's "
                "prefill does (gpt_oss/mxfp4/model_prefill.py:41-43)");
  if (cache_dtype != SNA_DTYPE_BF16 && cache_dtype != SNA_DTYPE_FP8_E4M3FN)
    return fail(SNA_ERR_INVALID_ARGUMENT, "qkv_norm_rope_store: unknown cache dtype %d", cache_dtype);
  const bool fp8 = cache_dtype == SNA_DTYPE_FP8_E4M3FN;
  if (n_tokens == 0) return SNA_OK;
  if (!qkv || !cos || !sin || !slots || !q_out || !k_cache || !v_cache || (fp8 && (!k_scale || !v_scale)))
    return fail(SNA_ERR_INVALID_ARGUMENT, "qkv_norm_rope_store: null pointer");
  if (!(eps >= 0.0f)) return fail(SNA_ERR_INVALID_ARGUMENT, "qkv_norm_rope_store: eps %g", (double)eps);
  if (!aligned(qkv, 16) || qkv_stride % 8 || !aligned(cos, 16) || !aligned(sin, 16) || rope_stride % 8 ||
      !aligned(q_out, 16) || !aligned(k_cache, 16) || !aligned(v_cache, 16) || (q_norm && (!aligned(q_norm, 16) ||
      !aligned(k_norm, 16))))
    return fail(SNA_ERR_INVALID_ARGUMENT, "qkv_norm_rope_store: tensors and row strides must be 16-byte aligned");
  const int32_t hpw = 64 / (head_dim / 8);
  const int64_t units = n_tokens * ((num_q_heads + 2 * num_kv_heads + hpw - 1) / hpw);
  const unsigned grid = (unsigned)std::min<int64_t>((units + 4 * 1 - 1) / (4 * 1), (int64_t)1 << 22);  // 4 waves x U
  const int64_t num_slots = num_blocks * page_size;
  hipStream_t s = (hipStream_t)stream;
#define SNA_QKV_LAUNCH(F, DD)                                                                                   \
  hipLaunchKernelGGL((qkv_norm_rope_store_kernel<F, DD>), dim3(grid), dim3(256), 0, s, (const uint16_t*)qkv,     \
                     qkv_stride, n_tokens, num_q_heads, num_kv_heads, (const uint16_t*)q_norm,                   \
                     (const uint16_t*)k_norm, eps, (const uint16_t*)cos, (const uint16_t*)sin, rope_stride, slots, \
                     (uint16_t*)q_out, (uint8_t*)k_cache, (uint8_t*)v_cache, k_scale, v_scale, num_slots, page_size)
  if (fp8 && head_dim == 128) SNA_QKV_LAUNCH(true, 128);
  else if (fp8) SNA_QKV_LAUNCH(true, 64);
  else if (head_dim == 128) SNA_QKV_LAUNCH(false, 128);
  else SNA_QKV_LAUNCH(false, 64);
#undef SNA_QKV_LAUNCH
  return check_launch("qkv_norm_rope_store");
}
