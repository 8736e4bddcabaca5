// KV-pool store kernels: quantize bf16 K/V (or MLA rows) to e4m3fn and scatter them to token slots.
//
// All are HBM-bound byte work: one pass over the input and one scattered write per token row. Lanes move 16 bytes of
// bf16 input and 8 bytes of fp8 output per access, so a token's head row is written by contiguous lanes.
#include "sna_device.h"
#include "sna_host.h"

namespace sna {

// ---------------------------------------------------------------------------------------------------------------
// MHA store. Thread = 8 consecutive elements of one (token, head) row of K and of V. MODE: kStoreBf16 (a copy),
// kStoreDiv (e4m3fn of x / s, s the dequantization scale) or kStoreMul (e4m3fn of bf16(x * m), m the reference's
// GPT-OSS quantization multiplier).
// ---------------------------------------------------------------------------------------------------------------
constexpr int kStoreBf16 = 0, kStoreDiv = 1, kStoreMul = 2;

template <int MODE>
__global__ __launch_bounds__(256) void kv_store_mha_kernel(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                                                           const int64_t* __restrict__ slots, int64_t n_tokens,
                                                           const float* __restrict__ k_scale,
                                                           const float* __restrict__ v_scale, uint8_t* __restrict__ kc,
                                                           uint8_t* __restrict__ vc, int64_t num_slots, int32_t G,
                                                           int32_t P, int32_t D) {
  const int32_t chunks = D / 8;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = n_tokens * G * chunks;
  if (idx >= total) return;
  const int32_t c = (int32_t)(idx % chunks);
  const int64_t th = idx / chunks;  // token * G + head
  const int32_t h = (int32_t)(th % G);
  const int64_t t = th / G;
  const int64_t slot = redirect_slot(slots[t], num_slots);
  const int64_t page = slot / P, off = slot % P;
  const int64_t dst_elem = ((page * G + h) * P + off) * D + (int64_t)c * 8;
  const int64_t src_elem = th * D + (int64_t)c * 8;
  const uint4 kin = ld16(k + src_elem);
  const uint4 vin = ld16(v + src_elem);
  if constexpr (MODE != kStoreBf16) {
    const float ks = k_scale[h], vs = v_scale[h];
    const uint32_t kw[4] = {kin.x, kin.y, kin.z, kin.w};
    const uint32_t vw[4] = {vin.x, vin.y, vin.z, vin.w};
    uint32_t ko[2] = {0, 0}, vo[2] = {0, 0};
    if constexpr (MODE == kStoreMul) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t kb = (kw[i >> 1] >> ((i & 1) * 16)) & 0xffffu;
        const uint32_t vb = (vw[i >> 1] >> ((i & 1) * 16)) & 0xffffu;
        ko[i >> 2] |= quantize_e4m3fn_mul(kb, ks) << ((i & 3) * 8);
        vo[i >> 2] |= quantize_e4m3fn_mul(vb, vs) << ((i & 3) * 8);
      }
    } else if (rcp_scale_ok(ks) && rcp_scale_ok(vs)) {
      const float rks = 1.0f / ks, rvs = 1.0f / vs;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ko[i >> 1] |= quantize_pair_e4m3fn_hw(kw[i], ks, rks) << ((i & 1) * 16);
        vo[i >> 1] |= quantize_pair_e4m3fn_hw(vw[i], vs, rvs) << ((i & 1) * 16);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t kb = (kw[i >> 1] >> ((i & 1) * 16)) & 0xffffu;
        const uint32_t vb = (vw[i >> 1] >> ((i & 1) * 16)) & 0xffffu;
        ko[i >> 2] |= quantize_e4m3fn(kb, ks) << ((i & 3) * 8);
        vo[i >> 2] |= quantize_e4m3fn(vb, vs) << ((i & 3) * 8);
      }
    }
    *reinterpret_cast<uint2*>(kc + dst_elem) = make_uint2(ko[0], ko[1]);
    *reinterpret_cast<uint2*>(vc + dst_elem) = make_uint2(vo[0], vo[1]);
  } else {
    *reinterpret_cast<uint4*>(kc + dst_elem * 2) = kin;
    *reinterpret_cast<uint4*>(vc + dst_elem * 2) = vin;
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Per-head absmax: pass 1 writes one partial max per (block, head), pass 2 reduces them into the scale.
// ---------------------------------------------------------------------------------------------------------------
constexpr int kAbsmaxBlocks = 256;

__global__ __launch_bounds__(256) void absmax_partial_kernel(const uint16_t* __restrict__ x, int64_t n_tokens,
                                                             int32_t H, int32_t D, float* __restrict__ partial) {
  const int32_t h = blockIdx.y;
  float m = 0.0f;
  const int32_t chunks = D / 8;
  const int64_t per_head = n_tokens * chunks;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < per_head; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i / chunks;
    const int32_t c = (int32_t)(i % chunks);
    const uint4 w = ld16(x + (t * H + h) * D + (int64_t)c * 8);
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      m = fmaxf(m, fabsf(bf16_bits_to_f32(ws[j] & 0xffffu)));
      m = fmaxf(m, fabsf(bf16_bits_to_f32(ws[j] >> 16)));
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  __shared__ float red[4];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    float r = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    partial[(int64_t)h * gridDim.x + blockIdx.x] = r;
  }
}

__global__ __launch_bounds__(64) void absmax_final_kernel(const float* __restrict__ partial, int32_t nblk,
                                                          float* __restrict__ scale_out) {
  const int32_t h = blockIdx.x;
  float m = 0.0f;
  for (int32_t i = threadIdx.x; i < nblk; i += 64) m = fmaxf(m, partial[(int64_t)h * nblk + i]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  if (threadIdx.x == 0) scale_out[h] = scale_from_absmax(m);
}

// ---------------------------------------------------------------------------------------------------------------
// MLA row store with a per-token scale. One wave per row; each lane holds up to 16 of the row's elements.
// ---------------------------------------------------------------------------------------------------------------
template <bool FP8>
__global__ __launch_bounds__(256) void kv_store_mla_kernel(const uint16_t* __restrict__ rows,
                                                           const int64_t* __restrict__ slots, int64_t n_tokens,
                                                           int32_t row_dim, uint8_t* __restrict__ cache,
                                                           float* __restrict__ row_scale, int64_t num_slots) {
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= n_tokens) return;
  const int lane = threadIdx.x & 63;
  const int32_t chunks = row_dim / 8;  // 8-element chunks per row
  const uint16_t* src = rows + t * row_dim;
  const int64_t slot = redirect_slot(slots[t], num_slots);
  // a lane owns chunks lane and lane + 64
  uint4 w0 = make_uint4(0, 0, 0, 0), w1 = make_uint4(0, 0, 0, 0);
  const bool has0 = lane < chunks, has1 = lane + 64 < chunks;
  if (has0) w0 = ld16(src + (int64_t)lane * 8);
  if (has1) w1 = ld16(src + (int64_t)(lane + 64) * 8);
  if constexpr (FP8) {
    float m = 0.0f;
    const uint32_t a[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      m = fmaxf(m, fabsf(bf16_bits_to_f32(a[j] & 0xffffu)));
      m = fmaxf(m, fabsf(bf16_bits_to_f32(a[j] >> 16)));
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    const float s = scale_from_absmax(m);
    uint8_t* dst = cache + slot * row_dim;
#pragma unroll
    for (int part = 0; part < 2; ++part) {
      if (part == 0 ? !has0 : !has1) continue;
      uint32_t o[2] = {0, 0};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t bits = (a[part * 4 + (i >> 1)] >> ((i & 1) * 16)) & 0xffffu;
        o[i >> 2] |= quantize_e4m3fn(bits, s) << ((i & 3) * 8);
      }
      *reinterpret_cast<uint2*>(dst + (int64_t)(lane + part * 64) * 8) = make_uint2(o[0], o[1]);
    }
    if (lane == 0) row_scale[slot] = s;
  } else {
    uint16_t* dst = reinterpret_cast<uint16_t*>(cache) + slot * row_dim;
    if (has0) *reinterpret_cast<uint4*>(dst + (int64_t)lane * 8) = w0;
    if (has1) *reinterpret_cast<uint4*>(dst + (int64_t)(lane + 64) * 8) = w1;
  }
}

// ---------------------------------------------------------------------------------------------------------------
// DSA 640-byte row store. One wave per row: lane l packs latent bytes [8l, 8l + 8) and, for l < 16, rope dims
// [4l, 4l + 4).
// ---------------------------------------------------------------------------------------------------------------
__device__ __forceinline__ int32_t dsa_latent_dim_of_byte(int32_t beta) {
  // inverse of byte = 256a + 2p + b for c = 256a + 128b + p (bytes relative to the latent field)
  const int32_t a = beta >> 8, rem = beta & 255;
  return (a << 8) + ((rem & 1) << 7) + (rem >> 1);
}

__global__ __launch_bounds__(256) void kv_store_dsa_kernel(const uint16_t* __restrict__ rows,
                                                           const int64_t* __restrict__ slots, int64_t n_tokens,
                                                           float kv_scale, uint8_t* __restrict__ cache,
                                                           int64_t num_rows) {
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= n_tokens) return;
  const int lane = threadIdx.x & 63;
  const int64_t slot = slots[t];
  if (slot < 0 || slot >= num_rows) return;
  const uint16_t* src = rows + t * 576;  // [k_pe 64 | latent 512]
  uint8_t* dst = cache + slot * 640;
  uint32_t o[2] = {0, 0};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int32_t c = dsa_latent_dim_of_byte(lane * 8 + i);
    o[i >> 2] |= quantize_e4m3fn(src[64 + c], kv_scale) << ((i & 3) * 8);
  }
  *reinterpret_cast<uint2*>(dst + 128 + lane * 8) = make_uint2(o[0], o[1]);
  if (lane < 16) {
    const uint2 w = ld8(src + lane * 4);
    const uint32_t e[4] = {w.x & 0xffffu, w.x >> 16, w.y & 0xffffu, w.y >> 16};
    uint32_t r0 = f32_to_bf16_bits(bf16_bits_to_f32(e[0]) / kv_scale) |
                  (f32_to_bf16_bits(bf16_bits_to_f32(e[1]) / kv_scale) << 16);
    uint32_t r1 = f32_to_bf16_bits(bf16_bits_to_f32(e[2]) / kv_scale) |
                  (f32_to_bf16_bits(bf16_bits_to_f32(e[3]) / kv_scale) << 16);
    *reinterpret_cast<uint2*>(dst + lane * 8) = make_uint2(r0, r1);
  }
}

__global__ void fp8_to_bf16_diag_kernel(const uint8_t* __restrict__ in, uint16_t* __restrict__ out, int64_t n) {
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i >= n) return;
  uint32_t w = 0;
  for (int j = 0; j < 4; ++j)
    if (i + j < n) w |= (uint32_t)in[i + j] << (8 * j);
  uint32_t lo, hi;
  fp8x4_to_bf16x4(w, lo, hi);
  const uint16_t r[4] = {(uint16_t)(lo & 0xffffu), (uint16_t)(lo >> 16), (uint16_t)(hi & 0xffffu),
                         (uint16_t)(hi >> 16)};
  for (int j = 0; j < 4; ++j)
    if (i + j < n) out[i + j] = r[j];
}

}  // namespace sna

using namespace sna;

extern "C" {

int sna_kv_store_mha(const void* k, const void* v, const int64_t* slots, int64_t n_tokens, const float* k_scale,
                     const float* v_scale, void* k_cache, void* v_cache, int64_t num_blocks, int32_t num_kv_heads,
                     int32_t page_size, int32_t head_dim, int32_t cache_dtype, void* stream) {
  ApiGuard guard;
  if (n_tokens < 0 || num_blocks < 1 || num_kv_heads < 1 || page_size < 1 || head_dim < 8 || head_dim % 8)
    return fail(SNA_ERR_INVALID_ARGUMENT, "kv_store_mha: bad sizes (n_tokens %lld, blocks %lld, heads %d, page %d, "
                "head_dim %d; head_dim must be a multiple of 8)", (long long)n_tokens, (long long)num_blocks,
                num_kv_heads, page_size, head_dim);
  if (cache_dtype != SNA_DTYPE_BF16 && cache_dtype != SNA_DTYPE_FP8_E4M3FN && cache_dtype != SNA_DTYPE_FP8_E4M3FN_MUL)
    return fail(SNA_ERR_INVALID_ARGUMENT, "kv_store_mha: unknown cache dtype %d", cache_dtype);
  if (n_tokens == 0) return SNA_OK;
  if (!k || !v || !slots || !k_cache || !v_cache)
    return fail(SNA_ERR_INVALID_ARGUMENT, "kv_store_mha: null pointer");
  const bool fp8 = cache_dtype != SNA_DTYPE_BF16;
  if (fp8 && (!k_scale || !v_scale)) return fail(SNA_ERR_INVALID_ARGUMENT, "kv_store_mha: FP8 cache needs k/v scales");
  if (!aligned(k, 16) || !aligned(v, 16) || !aligned(k_cache, 16) || !aligned(v_cache, 16))
    return fail(SNA_ERR_INVALID_ARGUMENT, "kv_store_mha: pointers must be 16-byte aligned");
  const int64_t total = n_tokens * num_kv_heads * (head_dim / 8);
  const dim3 grid((unsigned)((total + 255) / 256));
  hipStream_t s = (hipStream_t)stream;
  const int64_t num_slots = num_blocks * page_size;
  auto kernel = cache_dtype == SNA_DTYPE_FP8_E4M3FN_MUL ? kv_store_mha_kernel<kStoreMul>
                : cache_dtype == SNA_DTYPE_FP8_E4M3FN   ? kv_store_mha_kernel<kStoreDiv>
                                                        : kv_store_mha_kernel<kStoreBf16>;
  hipLaunchKernelGGL(kernel, grid, dim3(256), 0, s, (const uint16_t*)k, (const uint16_t*)v, slots, n_tokens, k_scale,
                     v_scale, (uint8_t*)k_cache, (uint8_t*)v_cache, num_slots, num_kv_heads, page_size, head_dim);
  return check_launch("kv_store_mha");
}

int64_t sna_absmax_workspace_bytes(int64_t n_tokens, int32_t num_heads) {
  (void)n_tokens;
  return (int64_t)kAbsmaxBlocks * (num_heads > 0 ? num_heads : 0) * (int64_t)sizeof(float);
}

int sna_kv_absmax_scale(const void* x, int64_t n_tokens, int32_t num_heads, int32_t head_dim, float* scale_out,
                        void* workspace, int64_t workspace_bytes, void* stream) {
  ApiGuard guard;
  if (n_tokens < 0 || num_heads < 1 || head_dim < 8 || head_dim % 8)
    return fail(SNA_ERR_INVALID_ARGUMENT, "kv_absmax_scale: bad sizes (n_tokens %lld, heads %d, head_dim %d)",
                (long long)n_tokens, num_heads, head_dim);
  if (!x || !scale_out || !workspace) return fail(SNA_ERR_INVALID_ARGUMENT, "kv_absmax_scale: null pointer");
  if (workspace_bytes < sna_absmax_workspace_bytes(n_tokens, num_heads))
    return fail(SNA_ERR_WORKSPACE, "kv_absmax_scale: workspace of %lld bytes, need %lld", (long long)workspace_bytes,
                (long long)sna_absmax_workspace_bytes(n_tokens, num_heads));
  if (!aligned(x, 16)) return fail(SNA_ERR_INVALID_ARGUMENT, "kv_absmax_scale: x must be 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(absmax_partial_kernel, dim3(kAbsmaxBlocks, num_heads), dim3(256), 0, s, (const uint16_t*)x,
                     n_tokens, num_heads, head_dim, (float*)workspace);
  int rc = check_launch("kv_absmax_scale");
  if (rc) return rc;
  hipLaunchKernelGGL(absmax_final_kernel, dim3(num_heads), dim3(64), 0, s, (const float*)workspace, kAbsmaxBlocks,
                     scale_out);
  return check_launch("kv_absmax_scale");
}

int sna_kv_store_mla(const void* rows, const int64_t* slots, int64_t n_tokens, int32_t row_dim, void* cache,
                     float* row_scale, int64_t num_slots, int32_t cache_dtype, void* stream) {
  ApiGuard guard;
  if (n_tokens < 0 || row_dim < 8 || row_dim % 8 || row_dim > 1024 || num_slots < 1)
    return fail(SNA_ERR_INVALID_ARGUMENT, "kv_store_mla: bad sizes (n_tokens %lld, row_dim %d (a multiple of 8, at "
                "most 1024), slots %lld)", (long long)n_tokens, row_dim, (long long)num_slots);
  if (cache_dtype != SNA_DTYPE_BF16 && cache_dtype != SNA_DTYPE_FP8_E4M3FN)
    return fail(SNA_ERR_INVALID_ARGUMENT, "kv_store_mla: unknown cache dtype %d", cache_dtype);
  if (n_tokens == 0) return SNA_OK;
  const bool fp8 = cache_dtype == SNA_DTYPE_FP8_E4M3FN;
  if (!rows || !slots || !cache || (fp8 && !row_scale))
    return fail(SNA_ERR_INVALID_ARGUMENT, "kv_store_mla: null pointer");
  if (!aligned(rows, 16) || !aligned(cache, 16))
    return fail(SNA_ERR_INVALID_ARGUMENT, "kv_store_mla: pointers must be 16-byte aligned");
  const dim3 grid((unsigned)((n_tokens + 3) / 4));
  hipStream_t s = (hipStream_t)stream;
  if (fp8)
    hipLaunchKernelGGL(kv_store_mla_kernel<true>, grid, dim3(256), 0, s, (const uint16_t*)rows, slots, n_tokens,
                       row_dim, (uint8_t*)cache, row_scale, num_slots);
  else
    hipLaunchKernelGGL(kv_store_mla_kernel<false>, grid, dim3(256), 0, s, (const uint16_t*)rows, slots, n_tokens,
                       row_dim, (uint8_t*)cache, row_scale, num_slots);
  return check_launch("kv_store_mla");
}

int sna_kv_store_dsa(const void* rows, const int64_t* slots, int64_t n_tokens, float kv_scale, void* cache,
                     int64_t num_rows, void* stream) {
  ApiGuard guard;
  if (n_tokens < 0 || num_rows < 1 || !(kv_scale > 0.0f))
    return fail(SNA_ERR_INVALID_ARGUMENT, "kv_store_dsa: bad arguments (n_tokens %lld, rows %lld, kv_scale %g)",
                (long long)n_tokens, (long long)num_rows, (double)kv_scale);
  if (n_tokens == 0) return SNA_OK;
  if (!rows || !slots || !cache) return fail(SNA_ERR_INVALID_ARGUMENT, "kv_store_dsa: null pointer");
  if (!aligned(rows, 8) || !aligned(cache, 16))
    return fail(SNA_ERR_INVALID_ARGUMENT, "kv_store_dsa: rows must be 8-byte and cache 16-byte aligned");
  const dim3 grid((unsigned)((n_tokens + 3) / 4));
  hipLaunchKernelGGL(kv_store_dsa_kernel, grid, dim3(256), 0, (hipStream_t)stream, (const uint16_t*)rows, slots,
                     n_tokens, kv_scale, (uint8_t*)cache, num_rows);
  return check_launch("kv_store_dsa");
}

int sna_diag_fp8_to_bf16(const uint8_t* in, uint16_t* out, int64_t n, void* stream) {
  ApiGuard guard;
  if (n < 0 || (n > 0 && (!in || !out))) return fail(SNA_ERR_INVALID_ARGUMENT, "diag_fp8_to_bf16: bad arguments");
  if (n == 0) return SNA_OK;
  const int64_t threads = (n + 3) / 4;
  hipLaunchKernelGGL(fp8_to_bf16_diag_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, in, out, n);
  return check_launch("diag_fp8_to_bf16");
}

}  // extern "C"
