// The writer half of the QKV step after the projection: per-head RMSNorm of Q and K (optional), rotate-half RoPE of
// Q and K, Q written out and K / V stored into the paged MHA pool (bf16, or e4m3fn with per-KV-head scales), in one
// pass over the projection's output.
//
// Heads are ordered [Q 0 .. Hq) [K 0 .. Hkv) [V 0 .. Hkv) as the fused projection lays them out. Every rounding step
// of the reference's torch path is kept: the norm rounds x * rsqrt(mean + eps) to bf16 and multiplies by the bf16
// gamma with a bf16 result; RoPE rounds each product and the sum to bf16. The sum of squares is fp32 in a fixed
// order (each square rounded, a lane's 8 in sequence, the head's lanes folded in halves) and 1 / sqrt is correctly
// rounded, the order and roundings the oracle states, so Q and both pools are bit-exact with it; a NaN output is a NaN
// where the reference's is (its bits are not fixed, there or here).
#include "sna_device.h"
#include "sna_host.h"

namespace sna {

// Two floats each rounded to bf16 (nearest even) and packed, lo in the low half, by one hardware conversion
// (v_cvt_pk_bf16_f32). Each half equals f32_to_bf16_bits of its input for every non-NaN input; a NaN stays a NaN
// (with its sign and leading payload bits: a NaN's bits are not fixed by the reference either, whose float to bf16
// conversion writes 0x7FC0 or 0xFFFF depending on the code path torch takes).
__device__ __forceinline__ uint32_t cvt_pk(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}
// The halves of a bf16 pair as floats.
__device__ __forceinline__ float lo_f(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float hi_f(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }

// The value of the lane `half` lanes away inside the head's lane group (lane ^ half). A 16-lane group (D = 128) is one
// DPP row, where a rotation by 8 is that exchange; other widths go through the LDS crossbar.
template <int HALF>
__device__ __forceinline__ uint32_t partner(uint32_t v) {
  if constexpr (HALF == 8) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xf, 0xf, true);  // row_ror:8
  else return (uint32_t)__shfl_xor((int)v, HALF, 64);
}

// The sum over the head's lane group, in every lane of it, folded in halves: lane i adds the lane HALF away, then
// HALF / 2, ..., 1 (every lane ends with the same bits, addition being commutative). DPP row rotations for a
// 16-lane group (rotations by 8, 4, 2, 1 pair the same lanes there), xor shuffles else. Every lane of the wave is
// active where it is called, so the rotations' bound_ctrl (what a disabled source lane gives) changes nothing; set,
// it lets each rotation fold into its add (v_add_f32_dpp).
template <int HALF>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (HALF == 8) {
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xf, 0xf, true));  // row_ror:8
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x124, 0xf, 0xf, true));  // row_ror:4
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x122, 0xf, 0xf, true));  // row_ror:2
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x121, 0xf, 0xf, true));  // row_ror:1
    return v;
  } else {
#pragma unroll
    for (int off = HALF; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
  }
}


// Lane layout: a head row of D bf16 is D / 8 lanes of 16 bytes (LPH lanes per head, 64 / LPH heads per wave), so
// every load and store is a 16-byte vector access. Lane j of a head holds elements 8 j .. 8 j + 7; its rotate-half
// partner (the lane LPH / 2 away) holds the elements D / 2 further on, fetched by one xor shuffle per dword. A
// workgroup takes one group of 64 / LPH consecutive heads (blockIdx.y; a head's type, Q, K or V, is fixed per
// LPH-lane group) over 4 U consecutive tokens (blockIdx.x), U per wave: the loads of the wave's U tokens are all issued
// before any is computed, and what depends only on the head (its gamma, its scale and that scale's reciprocal, its
// cache) is fetched once per wave.
template <bool FP8, int D, int U>
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
  const int32_t head = (int32_t)blockIdx.y * HPW + lane / LPH;
  const bool head_ok = head < heads;
  const bool is_q = head < Hq, is_k = !is_q && head < Hq + Hkv, roped = head < Hq + Hkv;
  const bool first = sub < HALF;
  // The wave's tokens are the same in every lane: from the wave index read once, every per-token address, the slot
  // and its page are scalar work; the lanes add only their head's and their own 16-byte offsets.
  const int32_t wave = __builtin_amdgcn_readfirstlane((int32_t)(threadIdx.x >> 6));
  const int64_t t0 = ((int64_t)blockIdx.x * 4 + wave) * U;
  const int32_t row_off = head * D + 8 * sub;  // the lane's offset in a token's projection row

  // this wave's U tokens: the head rows, the rotation rows (Q and K) and the slots, all loads in flight
  uint4 w[U], cw[U], sw[U];
  int64_t slot[U];
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const int64_t t = t0 + k;
    const bool live = t < n_tokens && head_ok;
    // the projection row is read once (non-temporal); cos / sin rows are read by every roped head group
    w[k] = live ? ld16_stream(qkv + t * qkv_stride + row_off) : make_uint4(0, 0, 0, 0);
    cw[k] = sw[k] = make_uint4(0, 0, 0, 0);
    if (live && roped) {
      cw[k] = ld16(cosv + t * rope_stride + 8 * sub);
      sw[k] = ld16(sinv + t * rope_stride + 8 * sub);
    }
    slot[k] = t < n_tokens ? slots[t] : 0;  // every token has a slot; a Q lane ignores it
  }
  // per head: the gamma (Q and K with the norm), the cache and its scale (K and V)
  float gf[8];  // the lane's 8 gamma elements as floats, converted once for the wave's tokens
#pragma unroll
  for (int e = 0; e < 8; ++e) gf[e] = 0.0f;
  if (q_norm && head_ok && roped) {  // q_norm: uniform, both gammas or neither
    const uint4 gw = ld16((is_q ? q_norm : k_norm) + 8 * sub);
    const uint32_t gg[4] = {gw.x, gw.y, gw.z, gw.w};
#pragma unroll
    for (int e2 = 0; e2 < 4; ++e2) {
      gf[2 * e2] = lo_f(gg[e2]);
      gf[2 * e2 + 1] = hi_f(gg[e2]);
    }
  }
  const int32_t h = head - Hq - (is_k ? 0 : Hkv);  // the KV head (K and V lanes)
  float scl = 1.0f, rs = 1.0f;
  bool rcp_ok = false;
  if (FP8 && head_ok && !is_q) {
    scl = is_k ? k_scale[h] : v_scale[h];
    rcp_ok = rcp_scale_ok(scl);
    rs = rcp_ok ? 1.0f / scl : 1.0f;
  }
  uint8_t* const cache = is_k ? kc : vc;
  const bool p_pow2 = (P & (P - 1)) == 0;  // uniform: the slot's page and offset by shifts
  const int p_shift = __builtin_ctz((uint32_t)P);
  const int64_t kv_off = ((int64_t)h * P) * D + 8 * sub;  // the lane's offset in a page (K and V lanes)

  const float sgn = first ? -1.0f : 1.0f;  // rotate-half: the first half takes the partner's value negated
  const bool kv_wave = !__all(is_q);       // the wave holds K or V heads (uniform)
  // _rms: gamma * (x32 * rsqrt(mean(x32^2) + eps)).to(bf16), rsqrt as 1 / sqrt (both correctly rounded). The sum of
  // squares: each square rounded (pow(2)), a lane's 8 summed in sequence, then the head's LPH lane sums folded in
  // halves (group_sum; every lane takes part in the shuffles). The U tokens' 1 / sqrt share one sequence: the head's
  // lanes are cut into U runs of LPH / U, run k computes token k's, and the lanes fetch the other tokens' results
  // from the runs that hold them.
  float inv[U];
#pragma unroll
  for (int k = 0; k < U; ++k) inv[k] = 1.0f;
  if (q_norm) {  // uniform
    static_assert(LPH % U == 0, "a head's lanes are cut into U equal runs");
    float ss[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const uint32_t xk[4] = {w[k].x, w[k].y, w[k].z, w[k].w};
      float sk = 0.0f;
      {
#pragma clang fp contract(off)
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
          const float a = lo_f(xk[e2]), b = hi_f(xk[e2]);
          sk = sk + a * a;
          sk = sk + b * b;
        }
      }
      ss[k] = group_sum<HALF>(sk);
    }
    constexpr int RUN = LPH / U;  // lanes per run
    const int run = sub / RUN;     // this lane computes token `run`'s
    float xs = ss[0];
#pragma unroll
    for (int k = 1; k < U; ++k) xs = run == k ? ss[k] : xs;
    // sqrtf: correctly rounded (__fsqrt_rn is the native one)
    const float mine = 1.0f / sqrtf(xs / (float)D + eps);
    if constexpr (U == 1) {
      inv[0] = mine;
    } else if constexpr (U == 2) {  // run 0 is the first half of the head's lanes: the partner lane holds the other
      const float other = __uint_as_float(partner<HALF>(__float_as_uint(mine)));
      inv[0] = first ? mine : other;
      inv[1] = first ? other : mine;
    } else {  // token k's from the lane of run k at this lane's place in its run
      const int src = lane - sub + sub % RUN;
#pragma unroll
      for (int k = 0; k < U; ++k) inv[k] = __shfl(mine, src + k * RUN, 64);
    }
  }
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const int64_t t = t0 + k;
    const bool live = t < n_tokens && head_ok;
    uint32_t xp[4] = {w[k].x, w[k].y, w[k].z, w[k].w};  // the lane's 8 elements as bf16 pairs
    if (q_norm && live && roped) {
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        const uint32_t n = cvt_pk(lo_f(xp[e2]) * inv[k], hi_f(xp[e2]) * inv[k]);
        xp[e2] = cvt_pk(gf[2 * e2] * lo_f(n), gf[2 * e2 + 1] * hi_f(n));
      }
    }
    float xf[8];  // the lane's elements as floats
#pragma unroll
    for (int e2 = 0; e2 < 4; ++e2) {
      xf[2 * e2] = lo_f(xp[e2]);
      xf[2 * e2 + 1] = hi_f(xp[e2]);
    }
    if (!live) continue;
    uint32_t ob[4];
    bool nan = false;  // a NaN among the lane's 8 output elements
    if (roped) {
      // rope(t) = t * c + cat(-t[D/2:], t[:D/2]) * s, every product and the sum rounded to bf16: each element's two
      // products by one pair conversion, the sum by the output's (sgn * r exact, so the FMA rounds once, as the sum)
      const uint32_t cc[4] = {cw[k].x, cw[k].y, cw[k].z, cw[k].w}, sc[4] = {sw[k].x, sw[k].y, sw[k].z, sw[k].w};
      // The partner's elements: it is a lane of the same head, so it is live and roped too, and active here. The
      // shuffles move floats, not pairs, so the partner's halves need no extraction of their own.
      float pf[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) pf[e] = __uint_as_float(partner<HALF>(__float_as_uint(xf[e])));
      float y[8];
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        const uint32_t r0 = cvt_pk(xf[2 * e2] * lo_f(cc[e2]), pf[2 * e2] * lo_f(sc[e2]));
        const uint32_t r1 = cvt_pk(xf[2 * e2 + 1] * hi_f(cc[e2]), pf[2 * e2 + 1] * hi_f(sc[e2]));
        y[2 * e2] = fmaf(sgn, hi_f(r0), lo_f(r0));
        y[2 * e2 + 1] = fmaf(sgn, hi_f(r1), lo_f(r1));
        ob[e2] = cvt_pk(y[2 * e2], y[2 * e2 + 1]);
      }
      if (FP8 && kv_wave) {  // uniform: only the FP8 store looks at NaNs, and a wave of Q heads stores none
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) nan |= (y[2 * e2] != y[2 * e2]) | (y[2 * e2 + 1] != y[2 * e2 + 1]);
      }
    } else {
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        ob[e2] = xp[e2];
        nan |= (xf[2 * e2] != xf[2 * e2]) | (xf[2 * e2 + 1] != xf[2 * e2 + 1]);
      }
    }
    if (is_q) {
      *reinterpret_cast<uint4*>(q_out + t * Hq * D + row_off) = make_uint4(ob[0], ob[1], ob[2], ob[3]);
      continue;
    }
    // K (rotated) or V into the pool at the token's slot, as the MHA store writes it: element
    // ((page * Hkv + h) * P + off) * D + 8 sub, the page's and the offset's part of it the same in every lane
    const int64_t sl = redirect_slot(slot[k], num_slots);
    const int64_t page = p_pow2 ? sl >> p_shift : sl / P;
    const int64_t off = p_pow2 ? sl & (P - 1) : sl % P;
    const int64_t dst = (page * Hkv * P + off) * D + kv_off;
    if constexpr (FP8) {
      uint32_t q8[2] = {0, 0};
      if (rcp_ok && !__any(nan)) {  // uniform: NaNs are rare, and only a wave that holds one takes their path
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2)
          q8[e2 >> 1] |= quantize_pair_e4m3fn_hw_nonan(lo_f(ob[e2]), hi_f(ob[e2]), scl, rs) << (16 * (e2 & 1));
      } else if (rcp_ok) {
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) q8[e2 >> 1] |= quantize_pair_e4m3fn_hw(ob[e2], scl, rs) << (16 * (e2 & 1));
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          q8[e >> 2] |= quantize_e4m3fn((ob[e >> 1] >> (16 * (e & 1))) & 0xffffu, scl) << (8 * (e & 3));
      }
      *reinterpret_cast<uint2*>(cache + dst) = make_uint2(q8[0], q8[1]);
    } else {
      *reinterpret_cast<uint4*>(cache + 2 * dst) = make_uint4(ob[0], ob[1], ob[2], ob[3]);
    }
  }
}

// Tokens per wave of a launch (their loads in flight together).
constexpr int kQkvTokensPerWave = 2;

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
  constexpr int U = kQkvTokensPerWave;
  const int32_t hpw = 64 / (head_dim / 8);
  const int64_t token_blocks = (n_tokens + 4 * U - 1) / (4 * U);  // 4 waves x U tokens
  if (token_blocks > INT32_MAX)
    return fail(SNA_ERR_INVALID_ARGUMENT, "qkv_norm_rope_store: %lld tokens is too many for one launch",
                (long long)n_tokens);
  const int64_t head_groups = (num_q_heads + 2 * (int64_t)num_kv_heads + hpw - 1) / hpw;
  if (head_groups > 65535)
    return fail(SNA_ERR_INVALID_ARGUMENT, "qkv_norm_rope_store: %lld heads is too many for one launch",
                (long long)num_q_heads + 2ll * num_kv_heads);
  const dim3 grid((unsigned)token_blocks, (unsigned)head_groups);
  const int64_t num_slots = num_blocks * page_size;
  hipStream_t s = (hipStream_t)stream;
#define SNA_QKV_LAUNCH(F, DD)                                                                                   \
  hipLaunchKernelGGL((qkv_norm_rope_store_kernel<F, DD, U>), grid, dim3(256), 0, s, (const uint16_t*)qkv,         \
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
