// GQA paged decode: split-K online softmax over the block table, MFMA for QK^T and PV, then a combine pass that adds
// the step's own token (and the sink), normalizes, and optionally stores the token into the pool.
//
// Work: one workgroup of 4 waves per (sequence, split, KV head). A wave takes 32-key tiles round-robin. The tile
// is two half-tiles of 16 keys, each inside one page (page_size is a multiple of 16).
//
// Lane roles in a wave (lane = 16 * g4 + li):
//   QK   S^T[key, head] = K[key, :] . Q[head, :]   with v_mfma_f32_16x16x32_bf16, M = 16 keys, N = 16 heads (the
//        group's heads, zero-padded), K = head_dim in steps of 32. Lane (g4, li) feeds key li's elements
//        [D/4 * g4, D/4 * (g4 + 1)) and head li's query elements over the same range. A and B use one K-index map,
//        so the contraction pairs them however the instruction orders K internally.
//   out  lane (g4, j) holds S^T[4 g4 + r, j], r = 0..3, for each half-tile: 8 keys of head j.
//   PV   O^T[d, head] = V^T[d, keys] . P^T[keys, head]   with v_mfma_f32_16x16x32_bf16, K = the tile's 32 keys,
//        ordered so that lane (g4, *) supplies keys {4 g4 .. 4 g4 + 3} of both half-tiles: exactly the probabilities
//        that lane already holds. So P never moves between lanes, and only V is transposed: lane (g4, li) loads
//        D/16 contiguous elements V[key, D/16 * li ...] of its 8 keys and regroups them in registers so that the
//        d-tile t operand holds V[8 keys, D/16 * li + t].
//   acc  lane (g4, j), d-tile t, row r accumulates O[head j, D/16 * (4 g4 + r) + t].
#include "sna_device.h"
#include "sna_host.h"

namespace sna {

struct GqaArgs {
  const uint16_t* q;
  const uint8_t* k_cache;
  const uint8_t* v_cache;
  const float* k_scale;
  const float* v_scale;
  const int32_t* table;
  int64_t table_stride;
  int32_t table_width;
  const int32_t* seq_lens;
  int32_t B, H, G, group, P;
  int64_t num_blocks;
  int32_t window;
  float sm_scale;
  int32_t split_tiles;
  int32_t n_work;
  float* ws_o;   // [n_work, H, D]  unnormalized partial outputs (V dequantized)
  float* ws_ml;  // [n_work, H, 2]  running max (log2 domain) and softmax sum
};

struct GqaCombineArgs {
  const uint16_t* q;
  const uint16_t* k_new;
  const uint16_t* v_new;
  const int64_t* new_slots;
  uint8_t* k_cache;
  uint8_t* v_cache;
  const float* k_scale;
  const float* v_scale;
  const float* sinks;
  const int32_t* seq_lens;
  int32_t B, H, G, group, P;
  int64_t num_blocks;
  int32_t window;
  float sm_scale;
  int32_t split_tiles;
  int32_t n_work;
  const float* ws_o;
  const float* ws_ml;
  uint16_t* out;
};

template <int NB>
__device__ __forceinline__ void load_bytes(const uint8_t* p, uint32_t (&dst)[NB / 4]) {
  static_assert(NB % 4 == 0, "whole dwords");
  if constexpr (NB % 16 == 0) {
#pragma unroll
    for (int i = 0; i < NB / 16; ++i) {
      const uint4 w = ld16(p + 16 * i);
      dst[4 * i] = w.x;
      dst[4 * i + 1] = w.y;
      dst[4 * i + 2] = w.z;
      dst[4 * i + 3] = w.w;
    }
  } else if constexpr (NB == 8) {
    const uint2 w = ld8(p);
    dst[0] = w.x;
    dst[1] = w.y;
  } else {
    static_assert(NB == 4, "4, 8 or a multiple of 16 bytes");
    dst[0] = ld4(p);
  }
}

template <int D, bool FP8, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void gqa_decode_kernel(GqaArgs a) {
  constexpr int ESZ = FP8 ? 1 : 2;
  constexpr int STEPS = D / 32;        // QK MFMA steps
  constexpr int KE = D / 4;            // K elements per lane per key
  constexpr int KB = KE * ESZ;         // K bytes per lane per key
  constexpr int VE = D / 16;           // V elements per lane per key (= PV d-tiles)
  constexpr int VB = VE * ESZ;         // V bytes per lane per key
  constexpr int DT = D / 16;           // PV d-tiles
  static_assert(D == 64 || D == 128, "head_dim 64 or 128");

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int g4 = lane >> 4;
  const int li = lane & 15;
  const int g = blockIdx.y;

  int32_t b, split;
  locate_work<32>(a.seq_lens, a.B, a.window, a.split_tiles, (int32_t)blockIdx.x, b, split);
  if (b < 0) return;  // uniform across the workgroup

  const int32_t L = a.seq_lens[b];
  const KeyRange kr = key_range(L, a.window);
  const int32_t t_first = kr.lo / 32 + split * a.split_tiles;
  const int32_t t_last = min(t_first + a.split_tiles, (kr.hi + 31) / 32);

  // Query operand: lane (g4, li) holds head li's elements [KE * g4, KE * g4 + KE) as packed bf16.
  uint32_t qv[STEPS][4];
  {
    const bool live = li < a.group;
    const int32_t h = g * a.group + (live ? li : 0);
    const uint16_t* qp = a.q + ((int64_t)b * a.H + h) * D + KE * g4;
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const uint4 w = live ? ld16(qp + 8 * s) : make_uint4(0, 0, 0, 0);
      qv[s][0] = w.x;
      qv[s][1] = w.y;
      qv[s][2] = w.z;
      qv[s][3] = w.w;
    }
  }

  const float kscale = FP8 ? a.k_scale[g] : 1.0f;
  const float vscale = FP8 ? a.v_scale[g] : 1.0f;
  const float qk_scale = a.sm_scale * kscale * kLog2e;
  const int64_t head_stride = (int64_t)a.P * D * ESZ;  // bytes of one (page, head) block
  const int32_t* trow = a.table + (int64_t)b * a.table_stride;

  float m_run = kNegBig;
  float l_run = 0.0f;
  f32x4_t acc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int32_t tile = t_first + wave; tile < t_last; tile += WAVES) {
    const int32_t T0 = tile * 32;
    // page of each half-tile (uniform across the wave); an entry outside the table or pool reads page 0, masked
    int32_t pg[2];
    bool pvalid[2];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int32_t col = (T0 + 16 * hf) / a.P;
      int32_t e = col < a.table_width ? trow[col] : -1;
      pvalid[hf] = e >= 0 && (int64_t)e < a.num_blocks;
      pg[hf] = pvalid[hf] ? e : 0;
    }
    const uint8_t* kbase[2];
    const uint8_t* vbase[2];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int64_t blk = ((int64_t)pg[hf] * a.G + g) * head_stride + (int64_t)((T0 + 16 * hf) % a.P) * D * ESZ;
      kbase[hf] = a.k_cache + blk;
      vbase[hf] = a.v_cache + blk;
    }

    // ---- loads ----
    uint32_t kraw[2][KB / 4];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) load_bytes<KB>(kbase[hf] + (int64_t)li * D * ESZ + KB * g4, kraw[hf]);
    uint32_t vraw[8][VB / 4];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int hf = e >> 2;
      const int key = 4 * g4 + (e & 3);
      load_bytes<VB>(vbase[hf] + (int64_t)key * D * ESZ + VB * li, vraw[e]);
    }

    // ---- S^T = K Q^T ----
    f32x4_t sc[2];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      f32x4_t s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < STEPS; ++st) {
        uint32_t op[4];
        if constexpr (FP8) {
          fp8x4_to_bf16x4(kraw[hf][2 * st], op[0], op[1]);
          fp8x4_to_bf16x4(kraw[hf][2 * st + 1], op[2], op[3]);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) op[i] = kraw[hf][4 * st + i];
        }
        s = mfma_16x16x32_bf16(op, qv[st], s);
      }
      sc[hf] = s;
    }

    // ---- mask and online softmax (log2 domain) ----
    float x[8];
    float tmax = -INFINITY;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int32_t pos = T0 + 16 * hf + 4 * g4 + r;
        const bool ok = pvalid[hf] && pos >= kr.lo && pos < kr.hi;
        const float v = ok ? sc[hf][r] * qk_scale : -INFINITY;
        x[4 * hf + r] = v;
        tmax = fmaxf(tmax, v);
      }
    }
    tmax = max_across_groups(tmax);
    const float m_new = fmaxf(m_run, tmax);
    const float alpha = exp2f(m_run - m_new);
    m_run = m_new;
    float p[8];
    float psum = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      p[i] = exp2f(x[i] - m_new);
      psum += p[i];
    }
    l_run = l_run * alpha + psum;
#pragma unroll
    for (int t = 0; t < DT; ++t) acc[t] *= alpha;
    uint32_t pop[4] = {pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]), pack_bf16x2(p[4], p[5]),
                       pack_bf16x2(p[6], p[7])};

    // ---- zero the V of keys outside the pages (a stale NaN there would survive p = 0) ----
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int hf = e >> 2;
      const int32_t pos = T0 + 16 * hf + 4 * g4 + (e & 3);
      const bool ok = pvalid[hf] && pos >= kr.lo && pos < kr.hi;
#pragma unroll
      for (int i = 0; i < VB / 4; ++i) vraw[e][i] = ok ? vraw[e][i] : 0u;
    }

    // ---- O^T += V^T P^T, one MFMA per 16-wide d-tile ----
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      uint32_t op[4];
      if constexpr (FP8) {
        // byte t of each key's VB-byte run
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          lo |= ((vraw[e][t >> 2] >> (8 * (t & 3))) & 0xffu) << (8 * e);
          hi |= ((vraw[e + 4][t >> 2] >> (8 * (t & 3))) & 0xffu) << (8 * e);
        }
        fp8x4_to_bf16x4(lo, op[0], op[1]);
        fp8x4_to_bf16x4(hi, op[2], op[3]);
      } else {
        // 16-bit element t of each key's run
#pragma unroll
        for (int pr = 0; pr < 4; ++pr) {
          const uint32_t e0 = (vraw[2 * pr][t >> 1] >> (16 * (t & 1))) & 0xffffu;
          const uint32_t e1 = (vraw[2 * pr + 1][t >> 1] >> (16 * (t & 1))) & 0xffffu;
          op[pr] = e0 | (e1 << 16);
        }
      }
      acc[t] = mfma_16x16x32_bf16(op, pop, acc[t]);
    }
  }

  // ---- merge the waves' partials in LDS and write this split's partial ----
  __shared__ float sm_o[WAVES][16][D + 1];
  __shared__ float sm_m[WAVES][16];
  __shared__ float sm_l[WAVES][16];
  const float l_tot = sum_across_groups(l_run);
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) sm_o[wave][li][VE * (4 * g4 + r) + t] = acc[t][r];
  if (g4 == 0) {
    sm_m[wave][li] = m_run;
    sm_l[wave][li] = l_tot;
  }
  __syncthreads();
  const int64_t wbase = (int64_t)blockIdx.x * a.H + (int64_t)g * a.group;
  for (int idx = threadIdx.x; idx < a.group * D; idx += 64 * WAVES) {
    const int j = idx / D, d = idx % D;
    float M = sm_m[0][j];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) M = fmaxf(M, sm_m[w][j]);
    float o = 0.0f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) o += exp2f(sm_m[w][j] - M) * sm_o[w][j][d];
    a.ws_o[(wbase + j) * D + d] = o * vscale;
    if (d == 0) {
      float l = 0.0f;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) l += exp2f(sm_m[w][j] - M) * sm_l[w][j];
      a.ws_ml[(wbase + j) * 2] = M;
      a.ws_ml[(wbase + j) * 2 + 1] = l;
    }
  }
}

// One workgroup per (sequence, KV head): the step's token in-band (and its store), the sink, the split merge.
template <int D, bool FP8>
__global__ __launch_bounds__(256) void gqa_combine_kernel(GqaCombineArgs a) {
  constexpr int ESZ = FP8 ? 1 : 2;
  const int b = blockIdx.x, g = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  __shared__ float sm_k[D], sm_v[D], sm_s[16];
  __shared__ int32_t sm_work[2];

  const int32_t L = a.seq_lens[b];
  if (wave == 0) {
    int32_t n = splits_of<32>(L, a.window, a.split_tiles);
    int32_t base = work_base_of<32>(a.seq_lens, b, a.window, a.split_tiles);
    if (base > a.n_work) base = a.n_work;
    if (base + n > a.n_work) n = a.n_work - base;
    if (lane == 0) {
      sm_work[0] = base;
      sm_work[1] = n;
    }
  }
  if (tid < D) {
    const int64_t src = ((int64_t)b * a.G + g) * D + tid;
    const uint32_t kb = a.k_new[src], vb = a.v_new[src];
    float kd, vd;
    if constexpr (FP8) {
      const float ks = a.k_scale[g], vs = a.v_scale[g];
      const uint32_t kq = quantize_e4m3fn(kb, ks), vq = quantize_e4m3fn(vb, vs);
      kd = e4m3fn_to_f32(kq) * ks;
      vd = e4m3fn_to_f32(vq) * vs;
      if (a.new_slots) {
        const int64_t slot = redirect_slot(a.new_slots[b], a.num_blocks * a.P);
        const int64_t dst = (((slot / a.P) * a.G + g) * a.P + slot % a.P) * D + tid;
        a.k_cache[dst] = (uint8_t)kq;
        a.v_cache[dst] = (uint8_t)vq;
      }
    } else {
      kd = bf16_bits_to_f32(kb);
      vd = bf16_bits_to_f32(vb);
      if (a.new_slots) {
        const int64_t slot = redirect_slot(a.new_slots[b], a.num_blocks * a.P);
        const int64_t dst = (((slot / a.P) * a.G + g) * a.P + slot % a.P) * D + tid;
        reinterpret_cast<uint16_t*>(a.k_cache)[dst] = (uint16_t)kb;
        reinterpret_cast<uint16_t*>(a.v_cache)[dst] = (uint16_t)vb;
      }
    }
    (void)ESZ;
    sm_k[tid] = kd;
    sm_v[tid] = vd;
  }
  __syncthreads();
  // score of the new token per head, in the log2 domain
  for (int j = wave; j < a.group; j += 4) {
    const int32_t h = g * a.group + j;
    const uint16_t* qp = a.q + ((int64_t)b * a.H + h) * D;
    float s = 0.0f;
    for (int d = lane; d < D; d += 64) s += bf16_bits_to_f32(qp[d]) * sm_k[d];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if (lane == 0) sm_s[j] = s * a.sm_scale * kLog2e;
  }
  __syncthreads();
  const int32_t base = sm_work[0], n = sm_work[1];
  for (int idx = tid; idx < a.group * D; idx += 256) {
    const int j = idx / D, d = idx % D;
    const int32_t h = g * a.group + j;
    const float s_new = sm_s[j];
    const float sink = a.sinks ? a.sinks[h] * kLog2e : -INFINITY;
    float M = fmaxf(s_new, sink);
    for (int32_t i = 0; i < n; ++i) M = fmaxf(M, a.ws_ml[((int64_t)(base + i) * a.H + h) * 2]);
    const float w_new = exp2f(s_new - M);
    float den = w_new + (a.sinks ? exp2f(sink - M) : 0.0f);
    float num = w_new * sm_v[d];
    for (int32_t i = 0; i < n; ++i) {
      const int64_t row = (int64_t)(base + i) * a.H + h;
      const float w = exp2f(a.ws_ml[row * 2] - M);
      den += w * a.ws_ml[row * 2 + 1];
      num += w * a.ws_o[row * D + d];
    }
    a.out[((int64_t)b * a.H + h) * D + d] = (uint16_t)f32_to_bf16_bits(num / den);
  }
}

template <int D, bool FP8>
static void launch_gqa(const GqaArgs& da, const GqaCombineArgs& ca, hipStream_t s) {
  if (da.n_work > 0)
    hipLaunchKernelGGL((gqa_decode_kernel<D, FP8, 4>), dim3(da.n_work, da.G), dim3(256), 0, s, da);
  hipLaunchKernelGGL((gqa_combine_kernel<D, FP8>), dim3(ca.B, ca.G), dim3(256), 0, s, ca);
}

}  // namespace sna

using namespace sna;

extern "C" int sna_paged_decode_gqa(const void* q, const void* k_cache, const void* v_cache, const float* k_scale,
                                    const float* v_scale, const int32_t* block_table, int64_t table_stride,
                                    int32_t table_width, const int32_t* seq_lens, const void* k_new,
                                    const void* v_new, const int64_t* new_slots, const float* sinks, int32_t window,
                                    float sm_scale, void* out, int32_t B, int32_t num_q_heads, int32_t num_kv_heads,
                                    int32_t head_dim, int32_t page_size, int64_t num_blocks, int32_t cache_dtype,
                                    const sna_split_plan* plan, void* workspace, int64_t workspace_bytes,
                                    void* stream) {
  ApiGuard guard;
  if (B < 0 || num_q_heads < 1 || num_kv_heads < 1 || num_q_heads % num_kv_heads)
    return fail(SNA_ERR_INVALID_ARGUMENT, "paged_decode_gqa: bad head counts (q %d, kv %d)", num_q_heads,
                num_kv_heads);
  const int32_t group = num_q_heads / num_kv_heads;
  if (group > 16)
    return fail(SNA_ERR_UNSUPPORTED, "paged_decode_gqa: GQA group %d > 16 (a workgroup covers 16 query heads)", group);
  if (head_dim != 64 && head_dim != 128)
    return fail(SNA_ERR_UNSUPPORTED, "paged_decode_gqa: head_dim %d (64 or 128 are built)", head_dim);
  if (page_size < 16 || page_size % 16)
    return fail(SNA_ERR_UNSUPPORTED, "paged_decode_gqa: page_size %d (a multiple of 16 is required)", page_size);
  if (cache_dtype != SNA_DTYPE_BF16 && cache_dtype != SNA_DTYPE_FP8_E4M3FN)
    return fail(SNA_ERR_INVALID_ARGUMENT, "paged_decode_gqa: unknown cache dtype %d", cache_dtype);
  if (window < 0 || table_width < 0 || table_stride < table_width || num_blocks < 1 || !(sm_scale > 0.0f))
    return fail(SNA_ERR_INVALID_ARGUMENT, "paged_decode_gqa: bad window %d, table %d/%lld, blocks %lld or scale %g",
                window, table_width, (long long)table_stride, (long long)num_blocks, (double)sm_scale);
  if (!plan || plan->tile != 32 || plan->split_tiles < 1 || plan->n_work < 0)
    return fail(SNA_ERR_INVALID_ARGUMENT, "paged_decode_gqa: missing or foreign split plan");
  if (B == 0) return SNA_OK;
  const bool fp8 = cache_dtype == SNA_DTYPE_FP8_E4M3FN;
  if (!q || !k_cache || !v_cache || !block_table || !seq_lens || !k_new || !v_new || !out ||
      (fp8 && (!k_scale || !v_scale)) || (plan->n_work > 0 && !workspace))
    return fail(SNA_ERR_INVALID_ARGUMENT, "paged_decode_gqa: null pointer");
  if (!aligned(q, 16) || !aligned(k_cache, 16) || !aligned(v_cache, 16))
    return fail(SNA_ERR_INVALID_ARGUMENT, "paged_decode_gqa: q and caches must be 16-byte aligned");
  const int64_t need = sna_decode_workspace_bytes(plan, num_q_heads, head_dim);
  if (plan->n_work > 0 && workspace_bytes < need)
    return fail(SNA_ERR_WORKSPACE, "paged_decode_gqa: workspace of %lld bytes, the plan needs %lld",
                (long long)workspace_bytes, (long long)need);
  if ((int64_t)plan->n_work > 2147483647LL || num_kv_heads > 65535 || B > 2147483647)
    return fail(SNA_ERR_INVALID_ARGUMENT, "paged_decode_gqa: grid too large");

  float* ws = (float*)workspace;
  const int64_t n_o = (int64_t)plan->n_work * num_q_heads * head_dim;
  GqaArgs da;
  da.q = (const uint16_t*)q;
  da.k_cache = (const uint8_t*)k_cache;
  da.v_cache = (const uint8_t*)v_cache;
  da.k_scale = k_scale;
  da.v_scale = v_scale;
  da.table = block_table;
  da.table_stride = table_stride;
  da.table_width = table_width;
  da.seq_lens = seq_lens;
  da.B = B;
  da.H = num_q_heads;
  da.G = num_kv_heads;
  da.group = group;
  da.P = page_size;
  da.num_blocks = num_blocks;
  da.window = window;
  da.sm_scale = sm_scale;
  da.split_tiles = plan->split_tiles;
  da.n_work = plan->n_work;
  da.ws_o = ws;
  da.ws_ml = ws ? ws + n_o : nullptr;

  GqaCombineArgs ca;
  ca.q = (const uint16_t*)q;
  ca.k_new = (const uint16_t*)k_new;
  ca.v_new = (const uint16_t*)v_new;
  ca.new_slots = new_slots;
  ca.k_cache = (uint8_t*)k_cache;
  ca.v_cache = (uint8_t*)v_cache;
  ca.k_scale = k_scale;
  ca.v_scale = v_scale;
  ca.sinks = sinks;
  ca.seq_lens = seq_lens;
  ca.B = B;
  ca.H = num_q_heads;
  ca.G = num_kv_heads;
  ca.group = group;
  ca.P = page_size;
  ca.num_blocks = num_blocks;
  ca.window = window;
  ca.sm_scale = sm_scale;
  ca.split_tiles = plan->split_tiles;
  ca.n_work = plan->n_work;
  ca.ws_o = da.ws_o;
  ca.ws_ml = da.ws_ml;
  ca.out = (uint16_t*)out;

  hipStream_t s = (hipStream_t)stream;
  if (head_dim == 128) {
    if (fp8) launch_gqa<128, true>(da, ca, s);
    else launch_gqa<128, false>(da, ca, s);
  } else {
    if (fp8) launch_gqa<64, true>(da, ca, s);
    else launch_gqa<64, false>(da, ca, s);
  }
  return check_launch("paged_decode_gqa");
}
