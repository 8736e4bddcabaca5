// Device helpers shared by the KV-store and decode kernels (gfx950 / CDNA4).
//
// Number formats follow the public specifications, not any library's code:
//   * bf16   : IEEE binary32 with the low 16 mantissa bits dropped; float -> bf16 rounds to nearest even.
//   * e4m3fn : OCP FP8 E4M3 ("fn": no infinities, one NaN code per sign, 0x7F / 0xFF). Bias 7, 3 mantissa bits,
//              max finite 448 = 1.75 * 2^8, min normal 2^-6, subnormals m * 2^-9.
// The store's arithmetic is  q = e4m3fn_RNE(clamp(float(x_bf16) / s, -448, 448))  with an IEEE-correct fp32
// division (the HIP default; this code is never built with fast-math).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sna {

constexpr float kFp8Max = 448.0f;
constexpr float kLog2e = 1.4426950408889634f;
// Running-max sentinel: finite, so exp2(m_old - m_new) never evaluates (-inf) - (-inf).
constexpr float kNegBig = -1.0e30f;
// The most splits a row may have (the combine passes hold one weight per split in LDS); the planner keeps to it.
constexpr int kMaxSplits = 64;
// The most rows of a GQA launch that sizes its splits on the device (their tile counts stay in one wave's registers),
// and the most 32-key tiles one of its rows may span (its split arithmetic divides through floats: ceil_div_small).
constexpr int kGqaDevSplitRows = 512;
constexpr int kGqaDevSplitMaxTiles = (1 << 17) - 1;
// The most keys one sparse (DSA) workgroup may resolve (their row ids live in the kernel's LDS); the planner keeps to it.
constexpr int kMlaMaxSplitKeys = 2048;
// The MLA / DSA stream split's counter block at the start of its workspace: per (row, head group) an arrival counter
// and a mask of merged latent blocks, then one count of finished workgroups, each in a 64-byte line of its own; zero
// at rest. The last line holds a sticky status word: a launch that finds a counter past what a clean block allows
// (an arrival past its row's count, or more finished workgroups than its grid) sets a bit there, and only the host's
// sna_stream_workspace_status clears it.
constexpr int kCounterStride = 16;        // int32 words between counters
constexpr int kStreamMaxCounters = 2047;  // (row, head group) pairs the block holds
constexpr int64_t kStreamCounterBytes = 256 * 1024;  // (2 * kStreamMaxCounters + 2) lines of 64 bytes
constexpr int kStreamDoneWord = kCounterStride * 2 * kStreamMaxCounters;
constexpr int kStreamStatusWord = kCounterStride * (2 * kStreamMaxCounters + 1);
static_assert((2 * kStreamMaxCounters + 2) * kCounterStride * 4 <= kStreamCounterBytes, "the counters fit");
// Polls of a row's arrival counter by a workgroup that published a partial, before it leaves the merge to others.
constexpr int kStreamWaitPolls = 96;
// A GQA plan's item map entry: row << 6 | split, with this bit set on a row's last item (its own token's split).
constexpr uint32_t kWorkLastSplit = 1u << 31;

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// float -> bf16 bits, round to nearest even; NaN -> 0x7FC0.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// float -> e4m3fn byte, round to nearest even. A magnitude that rounds above 448 (infinity included) and NaN give
// the NaN code with the input's sign, which is what a plain cast does; the store clamps first, so only NaN reaches
// that branch there.
__device__ __forceinline__ uint32_t f32_to_e4m3fn(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7fu;
  if (a < 0x3c800000u) {
    // |x| < 2^-6: the subnormal grid has step 2^-9. |x| * 512 is exact; rint rounds half to even. A result of 8 is
    // the encoding of 2^-6 (exponent 1, mantissa 0), so the carry into the exponent is free.
    return sign | (uint32_t)__builtin_rintf(__uint_as_float(a) * 512.0f);
  }
  // Normal: keep 3 of 23 mantissa bits with round-half-even at bit 20, then rebias the exponent 127 -> 7
  // (120 << 3 = 960). A mantissa carry moves into the exponent by the addition itself.
  uint32_t r = ((a + 0x7ffffu + ((a >> 20) & 1u)) >> 20) - 960u;
  if (r > 0x7eu) return sign | 0x7fu;
  return sign | r;
}

// e4m3fn byte -> float (exact).
__device__ __forceinline__ float e4m3fn_to_f32(uint32_t b) {
  const uint32_t sign = (b & 0x80u) << 24;
  const uint32_t e = (b >> 3) & 0xfu;
  const uint32_t m = b & 7u;
  if (e == 15u && m == 7u) return __uint_as_float(sign | 0x7fc00000u);
  if (e == 0u) return __uint_as_float(sign | __float_as_uint((float)m * 0.001953125f));  // m * 2^-9
  return __uint_as_float(sign | ((e + 120u) << 23) | (m << 20));
}

// An element v with |v| < 256 and at most 8 significant bits (a bf16 value times a power of two) as v = hi + lo / 16
// with hi its top 4 significant bits (truncated) and lo the next 4 times 16: both are e4m3fn values, exactly (but for
// elements below the e4m3fn normal range, which the conversion rounds).
__device__ __forceinline__ void split_q(float v, float& hi, float& lo) {
  hi = __uint_as_float(__float_as_uint(v) & 0xfff00000u);
  lo = (v - hi) * 16.0f;
}
// Four floats in the e4m3fn range to e4m3fn bytes 0..3 (round to nearest even; an exactly representable value is
// unchanged).
__device__ __forceinline__ uint32_t pack_e4m3fn_x4(float a, float b, float c, float d) {
  typedef short s16x2_t __attribute__((ext_vector_type(2)));
  s16x2_t w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32((s16x2_t){0, 0}, a, b, 1.0f, false);
  w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(w, c, d, 1.0f, true);
  return (uint32_t)(uint16_t)w[0] | ((uint32_t)(uint16_t)w[1] << 16);
}

// NaN-preserving clamp to the e4m3fn range: comparisons with NaN are false, so NaN passes through.
__device__ __forceinline__ float clamp_fp8(float x) {
  return x > kFp8Max ? kFp8Max : (x < -kFp8Max ? -kFp8Max : x);
}

// The store's quantizer: one bf16 element (its bits) and the dequantization scale s.
__device__ __forceinline__ uint32_t quantize_e4m3fn(uint32_t bf16_bits, float s) {
  return f32_to_e4m3fn(clamp_fp8(bf16_bits_to_f32(bf16_bits) / s));
}

// The GPT-OSS decode write (attention_decode.py:259-260): a bf16 element times the bf16 quantization multiplier m
// (the inverted checkpoint scale, gpt_oss/mxfp4/common.py:481-485), the product rounded to bf16 as a product of two
// bf16 tensors is, then clamped to +-448 (exact in bf16) and cast. The fp32 product of two bf16 values is exact (two
// 8-bit significands) outside the subnormal range, so the one rounding is the bf16 one. A NaN product is bf16's
// canonical NaN (0x7FC0), which casts to 0x7F.
__device__ __forceinline__ uint32_t quantize_e4m3fn_mul(uint32_t bf16_bits, float m) {
  const float p = bf16_bits_to_f32(bf16_bits) * m;
  return f32_to_e4m3fn(clamp_fp8(bf16_bits_to_f32(f32_to_bf16_bits(p))));
}

// quantize_e4m3fn of the two bf16 elements packed in `pair` (low half first), as a 16-bit pair of bytes (the low
// element's in the low byte), without a division per element: through the hardware conversion v_cvt_pk_fp8_f32
// (round to nearest even onto the OCP e4m3fn grid, subnormals included). The signed quotient x / s comes from x * rs held to +-1024 (beyond it the clamp
// gives +-448 whatever the rounding), corrected once by its exact FMA residual (Markstein's sequence: the correctly
// rounded quotient from the correctly rounded reciprocal rs = 1 / s), then clamped to +-448 by a median, so the
// conversion never overflows, and given x's sign (the residual's exact zero is +0, which would turn -0 into +0); a
// NaN element is written as its sign | 0x7F, as f32_to_e4m3fn writes it. s positive and normal (rcp_scale_ok).
__device__ __forceinline__ float with_sign_of(float mag, float x) {
  return __uint_as_float((__float_as_uint(mag) & 0x7fffffffu) | (__float_as_uint(x) & 0x80000000u));
}
// The bytes of two elements x0, x1 that are not NaN (bf16 values as floats): quantize_pair_e4m3fn_hw without its NaN
// step.
__device__ __forceinline__ uint32_t quantize_pair_e4m3fn_hw_nonan(float x0, float x1, float s, float rs) {
  const float q0 = __builtin_amdgcn_fmed3f(x0 * rs, -1024.0f, 1024.0f);
  const float q1 = __builtin_amdgcn_fmed3f(x1 * rs, -1024.0f, 1024.0f);
  const float y0 = with_sign_of(__builtin_amdgcn_fmed3f(fmaf(fmaf(-q0, s, x0), rs, q0), -kFp8Max, kFp8Max), x0);
  const float y1 = with_sign_of(__builtin_amdgcn_fmed3f(fmaf(fmaf(-q1, s, x1), rs, q1), -kFp8Max, kFp8Max), x1);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(y0, y1, 0, false) & 0xffffu;
}
__device__ __forceinline__ uint32_t quantize_pair_e4m3fn_hw(uint32_t pair, float s, float rs) {
  const float x0 = __uint_as_float(pair << 16), x1 = __uint_as_float(pair & 0xffff0000u);
  uint32_t b = quantize_pair_e4m3fn_hw_nonan(x0, x1, s, rs);
  if (x0 != x0) b = (b & 0xff00u) | ((pair >> 8) & 0x80u) | 0x7fu;
  if (x1 != x1) b = (b & 0x00ffu) | ((((pair >> 24) & 0x80u) | 0x7fu) << 8);
  return b;
}

// Whether quantize_pair_e4m3fn_hw serves the scale s (a positive normal float; otherwise use quantize_e4m3fn).
__device__ __forceinline__ bool rcp_scale_ok(float s) { return s >= 1.17549435e-38f && s <= 3.40282347e+38f; }

// The scale rule for per-head and per-token scales: absmax / 448, or 1 for an all-zero operand (whose bytes are then
// all zero), so no division by zero can happen.
__device__ __forceinline__ float scale_from_absmax(float amax) { return amax > 0.0f ? amax / kFp8Max : 1.0f; }

// Slot sanitising of the MHA pool write and of the MLA row write: a negative slot or one past the pool goes to
// slot 0, the reserved padding page.
__device__ __forceinline__ int64_t redirect_slot(int64_t slot, int64_t num_slots) {
  return (slot < 0 || slot >= num_slots) ? 0 : slot;
}

// ---- MFMA operand types (gfx950) ----
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Four e4m3fn bytes of a dword to four bf16 values in order (bytes 0..3). Exact: every e4m3fn value is a bf16 value.
__device__ __forceinline__ void fp8x4_to_bf16x4(uint32_t w, uint32_t& lo, uint32_t& hi) {
  bf16x2_t a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false);
  bf16x2_t b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true);
  lo = __builtin_bit_cast(uint32_t, a);
  hi = __builtin_bit_cast(uint32_t, b);
}

// ds_read_b64_tr_b8: in each 16-lane group the lanes' 8-byte chunks (8-byte aligned) form 8 rows of 16 bytes, row k
// being the chunks of lanes 2 k and 2 k + 1; lane j receives column j, so byte k of its result is byte j of row k.
__device__ __forceinline__ uint2 lds_read_tr8(const uint8_t* p) {
  typedef int32_t i32x2_t __attribute__((ext_vector_type(2)));
  const i32x2_t r = __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) i32x2_t*)(uint8_t*)p);
  return make_uint2((uint32_t)r.x, (uint32_t)r.y);
}

// ds_read_b64_tr_b16: in each 16-lane group the lanes' 8-byte chunks (8-byte aligned) form 4 rows of 16 16-bit
// elements, row k being the chunks of lanes 4 k .. 4 k + 3; lane j receives column j, so element k of its result
// (bits 16 k of the pair, low dword first) is element j of row k. (Measured on gfx950 with an in-bounds probe.)
__device__ __forceinline__ uint2 lds_read_tr16(const uint8_t* p) {
  typedef short s16x4_t_ __attribute__((ext_vector_type(4)));
  const s16x4_t_ r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4_t_*)(uint8_t*)p);
  return make_uint2((uint32_t)(uint16_t)r.x | ((uint32_t)(uint16_t)r.y << 16),
                    (uint32_t)(uint16_t)r.z | ((uint32_t)(uint16_t)r.w << 16));
}

// Loads straight into LDS (lane i's bytes land at LDS address m0 + size * i), written as inline assembly so that the
// compiler does not see them: it would otherwise drain every load in flight before any LDS read it cannot prove
// disjoint from them. Callers wait for them with wait_vmcnt, counting every such load they issued after the one they
// need. The buffer forms read through a buffer resource (a uniform base and size in SGPRs, a 32-bit offset per lane;
// reads past the size return zeros). The LDS address is wave-uniform (readfirstlane keeps it in an SGPR for m0); the
// s_nop covers the m0 write -> LDS-DMA hazard. The 16-byte forms carry the pool's pages, read once per decode: they
// are non-temporal (nt), which measured ~5% faster on the MLA gathers. The _cached forms are for pages that other
// workgroups read again soon (prefill: every query block of a request reads the same keys), kept in the L2.
typedef __attribute__((address_space(3))) void lds_ptr_t;
__device__ __forceinline__ uint32_t lds_address(const lds_ptr_t* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)p);
}
__device__ __forceinline__ void dma_buffer16(__amdgpu_buffer_rsrc_t r, uint32_t lds, uint32_t voff) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds" ::"s"(m0), "v"(voff), "s"(r)
               : "memory");
}
__device__ __forceinline__ void dma_buffer4(__amdgpu_buffer_rsrc_t r, uint32_t lds, uint32_t voff) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds" ::"s"(m0), "v"(voff), "s"(r)
               : "memory");
}
__device__ __forceinline__ void dma_global16(const void* src, uint32_t lds) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off nt" ::"s"(m0), "v"(src) : "memory");
}
__device__ __forceinline__ void dma_buffer16_cached(__amdgpu_buffer_rsrc_t r, uint32_t lds, uint32_t voff) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(m0), "v"(voff), "s"(r)
               : "memory");
}
__device__ __forceinline__ void dma_global16_cached(const void* src, uint32_t lds) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(m0), "v"(src) : "memory");
}
// XCD-aware order: workgroup i of a launch runs on XCD i mod 8 (an in-bounds probe of the XCC_ID register showed it
// for every workgroup of 256-, 512- and 1000-workgroup launches). xcd_order(i, n) deals the ids 0 .. n - 1 out so
// that each XCD takes a contiguous run of the logical order (the first n mod 8 XCDs one item more), so consecutive
// logical items share one XCD's L2. A bijection on [0, n) whatever the hardware's placement.
__device__ __forceinline__ uint32_t xcd_order(uint32_t i, uint32_t n) {
  const uint32_t per = n / 8, extra = n % 8, xcd = i % 8;
  return (xcd < extra ? xcd * (per + 1) : extra * (per + 1) + (xcd - extra) * per) + i / 8;
}
// Lane `src`'s 64-bit value (uniform), as two lane reads.
__device__ __forceinline__ int64_t readlane_i64(int64_t v, int src) {
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)(uint64_t)v, src);
  const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)((uint64_t)v >> 32), src);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// 4x4 byte transpose with v_perm_b32 (its 8 source bytes are {S1 bytes 0-3, S0 bytes 0-3} for selector values 0-7):
// byte r of w[e] becomes byte e of x[r].
__device__ __forceinline__ void transpose4x4_bytes(const uint32_t (&w)[4], uint32_t (&x)[4]) {
  const uint32_t t01l = __builtin_amdgcn_perm(w[1], w[0], 0x05010400u);  // w0.b0 w1.b0 w0.b1 w1.b1
  const uint32_t t01h = __builtin_amdgcn_perm(w[1], w[0], 0x07030602u);  // w0.b2 w1.b2 w0.b3 w1.b3
  const uint32_t t23l = __builtin_amdgcn_perm(w[3], w[2], 0x05010400u);
  const uint32_t t23h = __builtin_amdgcn_perm(w[3], w[2], 0x07030602u);
  x[0] = __builtin_amdgcn_perm(t23l, t01l, 0x05040100u);
  x[1] = __builtin_amdgcn_perm(t23l, t01l, 0x07060302u);
  x[2] = __builtin_amdgcn_perm(t23h, t01h, 0x05040100u);
  x[3] = __builtin_amdgcn_perm(t23h, t01h, 0x07060302u);
}

// Two floats to a packed pair of bf16 (round to nearest even), low half first.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  bf16x2_t v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ f32x4_t mfma_16x16x32_bf16(const uint32_t (&a)[4], const uint32_t (&b)[4], f32x4_t c) {
  typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
  u32x4_t av = {a[0], a[1], a[2], a[3]};
  u32x4_t bv = {b[0], b[1], b[2], b[3]};
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, av), __builtin_bit_cast(bf16x8_t, bv),
                                                  c, 0, 0, 0);
}

// FP8 (e4m3fn) A and B, K = 128; lane (g4, i) supplies row i of A and column i of B at the same 32 K positions, and the
// block scale 2^(scale_b - 127) of its B block (A's scale is 1).
typedef int32_t i32x8_t __attribute__((ext_vector_type(8)));
__device__ __forceinline__ f32x4_t mfma_16x16x128_fp8(const uint32_t (&a)[8], const uint32_t (&b)[8], f32x4_t c,
                                                     int32_t scale_b) {
  i32x8_t av, bv;
#pragma unroll
  for (int i = 0; i < 8; ++i) av[i] = (int32_t)a[i], bv[i] = (int32_t)b[i];
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, c, 0, 0, 0, 127, 0, scale_b);
}
__device__ __forceinline__ f32x4_t mfma_16x16x16_bf16(const uint32_t (&a)[2], const uint32_t (&b)[2], f32x4_t c) {
  typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
  u32x2_t av = {a[0], a[1]};
  u32x2_t bv = {b[0], b[1]};
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_t, av), __builtin_bit_cast(s16x4_t, bv),
                                                    c, 0, 0, 0);
}

// A wave-uniform read of memory no kernel of the launch writes (block tables, index lists, seq_lens): through the
// constant address space, so the compiler may use a scalar load, which waits on lgkmcnt and leaves the vector loads
// in flight alone.
template <typename T>
__device__ __forceinline__ T ld_const(const T* p) {
  return *(const __attribute__((address_space(4))) T*)(p);
}

// 16-, 8- and 4-byte global loads of raw bits.
__device__ __forceinline__ uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ uint2 ld8(const void* p) { return *reinterpret_cast<const uint2*>(p); }
__device__ __forceinline__ uint32_t ld4(const void* p) { return *reinterpret_cast<const uint32_t*>(p); }
// Loads of data read once (the KV pool's pages): non-temporal, so they do not displace what the caches hold for reuse
// (measured ~8% more HBM throughput on the paged gathers).
__device__ __forceinline__ uint4 ld16_stream(const void* p) {
  typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
  const u32x4_t w = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(w.x, w.y, w.z, w.w);
}
__device__ __forceinline__ uint2 ld8_stream(const void* p) {
  typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
  const u32x2_t w = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
  return make_uint2(w.x, w.y);
}
__device__ __forceinline__ uint32_t ld4_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
}

// Wave64 reductions across the four 16-lane groups (lanes l, l^16, l^32, l^48 hold the same MFMA column).
// Reductions over the 4 lanes li, li + 16, li + 32, li + 48 of a wave, through the permlane swaps (no LDS round
// trip): permlane32_swap of v with itself leaves lane l holding v[l] and v[l ^ 32] in its two results, and
// permlane16_swap v[l] and v[l ^ 16].
__device__ __forceinline__ float xor32_partner_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_across_groups(float v) {
  v = xor32_partner_max(v);
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_across_groups(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  const auto t = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(t[0]) + __uint_as_float(t[1]);
}
// Reductions over the 16 lanes of each 16-lane row, in VALU data-parallel moves (no LDS round trip): quad_perm
// [1,0,3,2] and [2,3,0,1] pair lanes within quads, row_half_mirror pairs a half-row's two quads, row_mirror the
// row's two halves. Each step combines two lanes that then hold the same value (the operations commute), so every
// lane of the row ends with the same bits.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_move<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v += dpp_move<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v += dpp_move<0x141>(v);  // row_half_mirror
  return v + dpp_move<0x140>(v);  // row_mirror
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_move<0xB1>(v));
  v = fmaxf(v, dpp_move<0x4E>(v));
  v = fmaxf(v, dpp_move<0x141>(v));
  return fmaxf(v, dpp_move<0x140>(v));
}
// Whole-wave reductions: across the four row groups, then within the row.
__device__ __forceinline__ float wave_max(float v) { return row16_max(max_across_groups(v)); }
__device__ __forceinline__ float wave_sum(float v) { return row16_sum(sum_across_groups(v)); }

// ceil(x / t) for x < 2^17 and 1 <= t < 2^17, with rt = 1 / t: the float quotient is within one of the exact one,
// and one correction each way makes it exact.
__device__ __forceinline__ uint32_t ceil_div_small(uint32_t x, uint32_t t, float rt) {
  uint32_t q = (uint32_t)((float)x * rt);
  if (q * t > x) --q;
  else if ((q + 1) * t <= x) ++q;
  return q + (q * t < x ? 1u : 0u);
}

// ---- split-K work decomposition ----
// Sequence b's keys from the pool are positions [lo_b, hi_b): hi_b = seq_len_b - 1 (the step's own token is attended
// in-band by the combine pass), lo_b = max(0, seq_len_b - window) for a sliding window of `window` keys (the new one
// included), else 0. Keys are processed in tiles of TILE positions aligned to absolute position multiples of TILE;
// a split is `split_tiles` consecutive tiles. The flattened work index runs over (sequence, split) in sequence order.
struct KeyRange {
  int32_t lo, hi;
};

__device__ __forceinline__ KeyRange key_range(int32_t seq_len, int32_t window) {
  KeyRange r;
  r.hi = seq_len - 1;
  r.lo = (window > 0 && seq_len - window > 0) ? seq_len - window : 0;
  if (r.hi < r.lo) r.hi = r.lo;
  return r;
}

template <int TILE>
__device__ __forceinline__ int32_t splits_of(int32_t seq_len, int32_t window, int32_t split_tiles) {
  if (seq_len <= 1) return 0;
  KeyRange r = key_range(seq_len, window);
  if (r.hi <= r.lo) return 0;
  int32_t t0 = r.lo / TILE, t1 = (r.hi + TILE - 1) / TILE;
  return (t1 - t0 + split_tiles - 1) / split_tiles;
}

// Wave-cooperative search: the (sequence, split) of flattened work index w, and the sequence's first work index.
// Every lane of the calling wave returns the same values; b = -1 when w is past the last split.
template <int TILE>
__device__ __forceinline__ void locate_work(const int32_t* __restrict__ seq_lens, int32_t B, int32_t window,
                                            int32_t split_tiles, int32_t w, int32_t& b_out, int32_t& split_out) {
  const int lane = threadIdx.x & 63;
  int32_t base = 0;
  b_out = -1;
  split_out = 0;
  for (int32_t b0 = 0; b0 < B; b0 += 64) {
    int32_t b = b0 + lane;
    int32_t n = b < B ? splits_of<TILE>(seq_lens[b], window, split_tiles) : 0;
    // inclusive scan over the wave
    int32_t incl = n;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      int32_t t = __shfl_up(incl, off, 64);
      if (lane >= off) incl += t;
    }
    int32_t excl = incl - n;
    const int32_t total = __builtin_amdgcn_readfirstlane(__shfl(incl, 63, 64));  // uniform loop exit
    if (w < base + total) {
      bool mine = (w >= base + excl) && (w < base + incl);
      unsigned long long ballot = __ballot(mine);
      int src = __ffsll((long long)ballot) - 1;
      int32_t e = __shfl(excl, src, 64);
      // the same for every lane: made scalar, so what is indexed by them stays in scalar registers
      b_out = __builtin_amdgcn_readfirstlane(b0 + src);
      split_out = __builtin_amdgcn_readfirstlane(w - base - e);
      return;
    }
    base += total;
  }
}

// First flattened work index of sequence b (same decomposition), computed by one wave.
template <int TILE>
__device__ __forceinline__ int32_t work_base_of(const int32_t* __restrict__ seq_lens, int32_t b, int32_t window,
                                                int32_t split_tiles) {
  const int lane = threadIdx.x & 63;
  int32_t acc = 0;
  for (int32_t b0 = 0; b0 < b; b0 += 64) {
    int32_t bb = b0 + lane;
    int32_t n = bb < b ? splits_of<TILE>(seq_lens[bb], window, split_tiles) : 0;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) n += __shfl_xor(n, off, 64);
    acc += n;
  }
  return acc;
}

}  // namespace sna
