// Absorbed-MLA decode (paged, per-token FP8 scale) and DSA sparse decode (index lists over 640-byte packed rows):
// split-K online softmax with all of a row's 16 heads in one wave, MFMA for QK^T and PV, and a combine pass that adds
// the step's own row, normalizes and (paged) stores the row.
//
// Row formats:
//   ROWS576  [latent 512 | k_pe 64] e4m3fn, one fp32 dequantization scale per token slot (row_scale).
//   ROWS640  [k_pe 64 bf16 | latent 512 e4m3fn, permuted], one per-tensor kv_scale. Latent dim c = 256a + 128b + p
//            sits at latent byte 256a + 2p + b.
//
// Lane roles (lane = 16 * g4 + li), 16-key tiles:
//   QK   S^T[key, head] = K[key, :] . Q[head, :]   v_mfma_f32_16x16x32_bf16, 18 steps over the 576 dims. Lane
//        (g4, li) feeds 144 (ROWS576) or 160 (ROWS640) bytes of key li's row, loaded straight from HBM, and head li's
//        query elements under the same K-index map.
//   PV   O^T[latent byte, head] = V^T[byte, keys] . P^T[keys, head]   v_mfma_f32_16x16x16_bf16, K = the 16 keys,
//        lane (g4, *) supplying keys 4 g4 .. 4 g4 + 3, the S^T rows it holds. The latent bytes of the tile go
//        through LDS. For d-tile (q, r), lane (g4, i) reads dword (64 q + 4 i) of rows 4 g4 .. 4 g4 + 3, transposes
//        the 4x4 bytes and feeds byte r of each.
//   acc  lane (g4, j) accumulates head j at latent bytes 64 q + 16 g4 + 4 r' + r  (q < 8, r < 4, r' < 4).
#include "sna_device.h"
#include "sna_host.h"

namespace sna {

enum { ROWS576 = 0, ROWS640 = 1 };

constexpr int kLatent = 512;
constexpr int kRope = 64;
constexpr int kLdsRow = 528;  // latent bytes of one key row in LDS, padded so row 4 apart hit other banks

struct MlaArgs {
  const uint16_t* ql;    // [B, H, 512]
  const uint16_t* qpe;   // [B, H, 64]
  const uint8_t* cache;  // rows
  const float* row_scale;
  float kv_scale;
  const int32_t* table;
  int64_t table_stride;
  int32_t table_width;
  const int32_t* seq_lens;   // paged
  const int32_t* indices;    // sparse [B, n_indices]
  int32_t n_indices;
  const int32_t* positions;  // sparse [B]
  int32_t B, H, P;
  int64_t num_blocks;
  float sm_scale;
  int32_t split_tiles, n_work;
  float* ws_o;   // [n_work, H, 512]  unnormalized partials, latent-byte order
  float* ws_ml;  // [n_work, H, 2]
};

struct MlaCombineArgs {
  const uint16_t* ql;
  const uint16_t* qpe;
  const uint16_t* own;  // [B, 576] bf16: ROWS576 [latent | rope], ROWS640 [rope | latent]
  const int64_t* new_slots;
  uint8_t* cache;
  float* row_scale;
  float kv_scale;
  const int32_t* seq_lens;
  int32_t n_indices;
  int32_t B, H, P;
  int64_t num_blocks;
  float sm_scale;
  int32_t split_tiles, n_work;
  const float* ws_o;
  const float* ws_ml;
  uint16_t* out;
  float* lse_out;
};

// latent byte (relative to the latent field) -> latent dim, for ROWS640
__device__ __forceinline__ int32_t latent_dim_of_byte(int32_t beta) {
  const int32_t a = beta >> 8, rem = beta & 255;
  return (a << 8) + ((rem & 1) << 7) + (rem >> 1);
}
// latent dim -> latent byte, for ROWS640
__device__ __forceinline__ int32_t latent_byte_of_dim(int32_t c) {
  const int32_t a = c >> 8, bb = (c >> 7) & 1, p = c & 127;
  return (a << 8) + 2 * p + bb;
}

template <int FMT>
struct RowFmt;
template <>
struct RowFmt<ROWS576> {
  static constexpr int kRowBytes = 576;
  static constexpr int kLaneChunks = 9;  // 16-byte chunks per lane per key
};
template <>
struct RowFmt<ROWS640> {
  static constexpr int kRowBytes = 640;
  static constexpr int kLaneChunks = 10;
};

// Byte offset within the row of chunk c of lane group g4.
template <int FMT>
__device__ __forceinline__ int chunk_offset(int g4, int c) {
  if constexpr (FMT == ROWS576) {
    return 144 * g4 + 16 * c;
  } else {
    return c < 2 ? 32 * g4 + 16 * c : 128 + 128 * g4 + 16 * (c - 2);
  }
}

template <int FMT, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void mla_decode_kernel(MlaArgs a) {
  constexpr int NCH = RowFmt<FMT>::kLaneChunks;
  constexpr int ROWB = RowFmt<FMT>::kRowBytes;
  constexpr bool SPARSE = FMT == ROWS640;

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int g4 = lane >> 4;
  const int li = lane & 15;
  const int hg = blockIdx.y;  // 16-head group

  __shared__ __attribute__((aligned(16))) uint8_t sm_lat[WAVES][16 * kLdsRow];
  __shared__ float sm_o[16][kLatent + 4];
  __shared__ float sm_m[WAVES][16];
  __shared__ float sm_l[WAVES][16];

  // Paged: keys are positions [0, seq_len - 1). Sparse: keys are index-list entries [0, n_indices), modelled as a
  // "sequence" of n_indices + 1 so the same decomposition applies (every row has the same split count).
  int32_t b = -1, split = 0;
  if constexpr (SPARSE) {
    const int32_t per = splits_of<16>(a.n_indices + 1, 0, a.split_tiles);
    const int32_t w = blockIdx.x;
    if (per > 0 && w < per * a.B) {
      b = w / per;
      split = w % per;
    }
  } else {
    locate_work<16>(a.seq_lens, a.B, 0, a.split_tiles, (int32_t)blockIdx.x, b, split);
  }
  if (b < 0) return;

  int32_t klo = 0, khi;
  if constexpr (SPARSE) {
    khi = a.n_indices;
  } else {
    khi = a.seq_lens[b] - 1;
  }
  const int32_t t_first = split * a.split_tiles;
  const int32_t t_last = min(t_first + a.split_tiles, (khi + 15) / 16);

  // ---- query operand: 18 steps x 8 elements for head (16 hg + li) ----
  uint32_t qv[18][4];
  {
    const int32_t h = 16 * hg + li;
    const bool live = h < a.H;
    const uint16_t* qlp = a.ql + ((int64_t)b * a.H + (live ? h : 0)) * kLatent;
    const uint16_t* qpp = a.qpe + ((int64_t)b * a.H + (live ? h : 0)) * kRope;
#pragma unroll
    for (int s = 0; s < 18; ++s) {
      uint4 w = make_uint4(0, 0, 0, 0);
      if (live) {
        if constexpr (FMT == ROWS576) {
          const int dim = 144 * g4 + 8 * s;  // natural order: latent then rope
          w = dim < kLatent ? ld16(qlp + dim) : ld16(qpp + (dim - kLatent));
        } else {
          if (s < 2) {
            w = ld16(qpp + 16 * g4 + 8 * s);
          } else {
            uint32_t e[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) e[i] = qlp[latent_dim_of_byte(128 * g4 + 8 * (s - 2) + i)];
            w = make_uint4(e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16), e[6] | (e[7] << 16));
          }
        }
      }
      qv[s][0] = w.x;
      qv[s][1] = w.y;
      qv[s][2] = w.z;
      qv[s][3] = w.w;
    }
  }

  const float base_scale = a.sm_scale * kLog2e * (SPARSE ? a.kv_scale : 1.0f);
  const int32_t* trow = a.table + (int64_t)b * a.table_stride;
  const int64_t n_rows = a.num_blocks * a.P;
  int32_t qpos = 0;
  if constexpr (SPARSE) qpos = a.positions[b];

  float m_run = kNegBig;
  float l_run = 0.0f;
  f32x4_t acc[8][4];
#pragma unroll
  for (int q = 0; q < 8; ++q)
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[q][r] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  uint8_t* lds = sm_lat[wave];

  for (int32_t tile = t_first + wave; tile < t_last; tile += WAVES) {
    const int32_t T0 = tile * 16;
    // ---- the row of key li (this lane's load) and the validity of every key of the tile ----
    int64_t row = 0;
    bool kvalid;
    if constexpr (SPARSE) {
      const int32_t k = T0 + li;
      const int32_t pos = k < khi ? a.indices[(int64_t)b * a.n_indices + k] : -1;
      kvalid = false;
      if (pos >= 0 && pos <= qpos) {
        const int32_t blk = pos / a.P;
        if (blk < a.table_width) {
          const int32_t e = trow[blk];
          if (e >= 0 && (int64_t)e < a.num_blocks) {
            row = (int64_t)e * a.P + pos % a.P;
            kvalid = row < n_rows;
            if (!kvalid) row = 0;
          }
        }
      }
    } else {
      const int32_t col = T0 / a.P;
      const int32_t e = col < a.table_width ? trow[col] : -1;
      const bool pv = e >= 0 && (int64_t)e < a.num_blocks;
      const int32_t pos = T0 + li;
      kvalid = pv && pos >= klo && pos < khi;
      row = (pv ? (int64_t)e * a.P : 0) + (T0 % a.P) + li;
    }
    const uint32_t vmask = (uint32_t)(__ballot(kvalid) & 0xffffull);  // bit k: key k of the tile is valid

    // ---- loads: NCH 16-byte chunks of row `row` ----
    uint32_t raw[NCH][4];
    const uint8_t* rp = a.cache + row * ROWB;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const uint4 w = ld16(rp + chunk_offset<FMT>(g4, c));
      raw[c][0] = kvalid ? w.x : 0u;
      raw[c][1] = kvalid ? w.y : 0u;
      raw[c][2] = kvalid ? w.z : 0u;
      raw[c][3] = kvalid ? w.w : 0u;
    }
    float kscale[4] = {1.f, 1.f, 1.f, 1.f};
    if constexpr (!SPARSE) {
      // per-token scales of keys 4 g4 .. 4 g4 + 3: four consecutive slots of one page
      const int32_t col = T0 / a.P;
      const int32_t e = col < a.table_width ? trow[col] : -1;
      const bool pv = e >= 0 && (int64_t)e < a.num_blocks;
      const int64_t srow = (pv ? (int64_t)e * a.P : 0) + (T0 % a.P) + 4 * g4;
      const float4 s4 = *reinterpret_cast<const float4*>(a.row_scale + srow);
      kscale[0] = s4.x;
      kscale[1] = s4.y;
      kscale[2] = s4.z;
      kscale[3] = s4.w;
    }

    // ---- latent bytes to LDS for the PV transpose ----
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      int lat;  // latent byte offset of the chunk, or -1
      if constexpr (FMT == ROWS576) {
        const int off = chunk_offset<FMT>(g4, c);
        lat = off < kLatent ? off : -1;
      } else {
        lat = c < 2 ? -1 : 128 * g4 + 16 * (c - 2);
      }
      if (lat >= 0)
        *reinterpret_cast<uint4*>(lds + li * kLdsRow + lat) = make_uint4(raw[c][0], raw[c][1], raw[c][2], raw[c][3]);
    }

    // ---- S^T = K Q^T ----
    f32x4_t sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 18; ++s) {
      uint32_t op[4];
      if constexpr (FMT == ROWS576) {
        const int c = s >> 1, hf = s & 1;
        fp8x4_to_bf16x4(raw[c][2 * hf], op[0], op[1]);
        fp8x4_to_bf16x4(raw[c][2 * hf + 1], op[2], op[3]);
      } else {
        if (s < 2) {
#pragma unroll
          for (int i = 0; i < 4; ++i) op[i] = raw[s][i];
        } else {
          const int c = 2 + ((s - 2) >> 1), hf = (s - 2) & 1;
          fp8x4_to_bf16x4(raw[c][2 * hf], op[0], op[1]);
          fp8x4_to_bf16x4(raw[c][2 * hf + 1], op[2], op[3]);
        }
      }
      sc = mfma_16x16x32_bf16(op, qv[s], sc);
    }

    // ---- mask, online softmax ----
    float x[4];
    float tmax = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool ok = (vmask >> (4 * g4 + r)) & 1u;
      const float v = ok ? sc[r] * base_scale * kscale[r] : -INFINITY;
      x[r] = v;
      tmax = fmaxf(tmax, v);
    }
    tmax = max_across_groups(tmax);
    const float m_new = fmaxf(m_run, tmax);
    const float alpha = exp2f(m_run - m_new);
    m_run = m_new;
    float p[4], psum = 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      p[r] = exp2f(x[r] - m_new);
      psum += p[r];
    }
    l_run = l_run * alpha + psum;
    if (alpha != 1.0f) {
#pragma unroll
      for (int q = 0; q < 8; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[q][r] *= alpha;
    }
    // V is dequantized through P: p' = p * scale(key) (a masked key has p = 0 and a zeroed row)
    const bool ok0 = (vmask >> (4 * g4)) & 1u, ok1 = (vmask >> (4 * g4 + 1)) & 1u;
    const bool ok2 = (vmask >> (4 * g4 + 2)) & 1u, ok3 = (vmask >> (4 * g4 + 3)) & 1u;
    const uint32_t pop[2] = {pack_bf16x2(ok0 ? p[0] * kscale[0] : 0.f, ok1 ? p[1] * kscale[1] : 0.f),
                             pack_bf16x2(ok2 ? p[2] * kscale[2] : 0.f, ok3 ? p[3] * kscale[3] : 0.f)};

    // ---- O^T += V^T P^T over 32 d-tiles ----
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      uint32_t w[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) w[e] = *reinterpret_cast<const uint32_t*>(lds + (4 * g4 + e) * kLdsRow + 64 * q + 4 * li);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t xr = ((w[0] >> (8 * r)) & 0xffu) | (((w[1] >> (8 * r)) & 0xffu) << 8) |
                            (((w[2] >> (8 * r)) & 0xffu) << 16) | (((w[3] >> (8 * r)) & 0xffu) << 24);
        uint32_t op[2];
        fp8x4_to_bf16x4(xr, op[0], op[1]);
        acc[q][r] = mfma_16x16x16_bf16(op, pop, acc[q][r]);
      }
    }
    __builtin_amdgcn_wave_barrier();
  }

  // ---- merge the waves: common max, then sum the rescaled accumulators through LDS ----
  const float l_tot = sum_across_groups(l_run);
  if (g4 == 0) {
    sm_m[wave][li] = m_run;
    sm_l[wave][li] = l_tot;
  }
  __syncthreads();
  float M = sm_m[0][li];
#pragma unroll
  for (int w = 1; w < WAVES; ++w) M = fmaxf(M, sm_m[w][li]);
  const float f = exp2f(m_run - M);
#pragma unroll
  for (int w = 0; w < WAVES; ++w) {
    if (wave == w) {
#pragma unroll
      for (int q = 0; q < 8; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) {
            const int beta = 64 * q + 16 * g4 + 4 * rr + r;
            const float v = acc[q][r][rr] * f;
            if (w == 0) sm_o[li][beta] = v;
            else sm_o[li][beta] += v;
          }
    }
    __syncthreads();
  }
  const int64_t wrow = (int64_t)blockIdx.x * a.H + 16 * hg;
  const float oscale = SPARSE ? a.kv_scale : 1.0f;
  const int nh = min(16, a.H - 16 * hg);
  for (int idx = threadIdx.x; idx < nh * kLatent; idx += 64 * WAVES) {
    const int j = idx / kLatent, beta = idx % kLatent;
    a.ws_o[(wrow + j) * kLatent + beta] = sm_o[j][beta] * oscale;
  }
  if (threadIdx.x < nh) {
    const int j = threadIdx.x;
    float Mj = sm_m[0][j];
    for (int w = 1; w < WAVES; ++w) Mj = fmaxf(Mj, sm_m[w][j]);
    float l = 0.0f;
    for (int w = 0; w < WAVES; ++w) l += exp2f(sm_m[w][j] - Mj) * sm_l[w][j];
    a.ws_ml[(wrow + j) * 2] = Mj;
    a.ws_ml[(wrow + j) * 2 + 1] = l;
  }
}

// One workgroup per (sequence, 16-head group): the own row in-band (and its store), then the split merge.
template <int FMT>
__global__ __launch_bounds__(256) void mla_combine_kernel(MlaCombineArgs a) {
  constexpr bool SPARSE = FMT == ROWS640;
  const int b = blockIdx.x, hg = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  __shared__ float sm_row[576];  // the own row, dequantized, natural order [latent 512 | rope 64]
  __shared__ float sm_s[16];
  __shared__ float sm_red[4];
  __shared__ int32_t sm_work[2];
  const int nh = min(16, a.H - 16 * hg);

  if (wave == 0) {
    int32_t n, base;
    if constexpr (SPARSE) {
      n = splits_of<16>(a.n_indices + 1, 0, a.split_tiles);
      base = b * n;
    } else {
      n = splits_of<16>(a.seq_lens[b], 0, a.split_tiles);
      base = work_base_of<16>(a.seq_lens, b, 0, a.split_tiles);
    }
    if (base > a.n_work) base = a.n_work;
    if (base + n > a.n_work) n = a.n_work - base;
    if (lane == 0) {
      sm_work[0] = base;
      sm_work[1] = n;
    }
  }
  // ---- own row: quantize -> dequantize (and store) ----
  const uint16_t* own = a.own + (int64_t)b * 576;
  if constexpr (!SPARSE) {
    float m = 0.0f;
    for (int i = tid; i < 576; i += 256) m = fmaxf(m, fabsf(bf16_bits_to_f32(own[i])));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if (lane == 0) sm_red[wave] = m;
    __syncthreads();
    const float s = scale_from_absmax(fmaxf(fmaxf(sm_red[0], sm_red[1]), fmaxf(sm_red[2], sm_red[3])));
    const bool store = a.new_slots != nullptr && hg == 0;
    const int64_t slot = store ? redirect_slot(a.new_slots[b], a.num_blocks * a.P) : 0;
    for (int i = tid; i < 576; i += 256) {
      const uint32_t qb = quantize_e4m3fn(own[i], s);
      sm_row[i] = e4m3fn_to_f32(qb) * s;
      if (store) a.cache[slot * 576 + i] = (uint8_t)qb;
    }
    if (store && tid == 0) a.row_scale[slot] = s;
  } else {
    // [rope 64 | latent 512] in, as the 640-byte row would hold it, dequantized back with kv_scale
    for (int i = tid; i < 576; i += 256) {
      const uint32_t bits = own[i];
      float v;
      if (i < kRope) {
        v = bf16_bits_to_f32(f32_to_bf16_bits(bf16_bits_to_f32(bits) / a.kv_scale)) * a.kv_scale;
        sm_row[kLatent + i] = v;
      } else {
        v = e4m3fn_to_f32(quantize_e4m3fn(bits, a.kv_scale)) * a.kv_scale;
        sm_row[i - kRope] = v;
      }
    }
  }
  __syncthreads();
  // ---- the own row's score per head (log2 domain) ----
  for (int j = wave; j < nh; j += 4) {
    const int32_t h = 16 * hg + j;
    const uint16_t* qlp = a.ql + ((int64_t)b * a.H + h) * kLatent;
    const uint16_t* qpp = a.qpe + ((int64_t)b * a.H + h) * kRope;
    float s = 0.0f;
    for (int d = lane; d < kLatent; d += 64) s += bf16_bits_to_f32(qlp[d]) * sm_row[d];
    s += bf16_bits_to_f32(qpp[lane]) * sm_row[kLatent + lane];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if (lane == 0) sm_s[j] = s * a.sm_scale * kLog2e;
  }
  __syncthreads();
  const int32_t base = sm_work[0], n = sm_work[1];
  for (int idx = tid; idx < nh * kLatent; idx += 256) {
    const int j = idx / kLatent, c = idx % kLatent;
    const int32_t h = 16 * hg + j;
    const int beta = SPARSE ? latent_byte_of_dim(c) : c;
    const float s_new = sm_s[j];
    float M = s_new;
    for (int32_t i = 0; i < n; ++i) M = fmaxf(M, a.ws_ml[((int64_t)(base + i) * a.H + h) * 2]);
    const float w_new = exp2f(s_new - M);
    float den = w_new, num = w_new * sm_row[c];
    for (int32_t i = 0; i < n; ++i) {
      const int64_t r = (int64_t)(base + i) * a.H + h;
      const float w = exp2f(a.ws_ml[r * 2] - M);
      den += w * a.ws_ml[r * 2 + 1];
      num += w * a.ws_o[r * kLatent + beta];
    }
    a.out[((int64_t)b * a.H + h) * kLatent + c] = (uint16_t)f32_to_bf16_bits(num / den);
    if (a.lse_out && c == 0) a.lse_out[(int64_t)b * a.H + h] = (M + log2f(den)) * 0.6931471805599453f;
  }
}

}  // namespace sna

using namespace sna;

extern "C" int sna_mla_decode(const void* ql_nope, const void* q_pe, const void* cache, const float* row_scale,
                              const int32_t* block_table, int64_t table_stride, int32_t table_width,
                              const int32_t* seq_lens, const void* compact_new, const int64_t* new_slots,
                              float sm_scale, void* out, int32_t B, int32_t num_heads, int32_t page_size,
                              int64_t num_blocks, int32_t cache_dtype, const sna_split_plan* plan, void* workspace,
                              int64_t workspace_bytes, void* stream) {
  ApiGuard guard;
  if (cache_dtype != SNA_DTYPE_FP8_E4M3FN)
    return fail(SNA_ERR_UNSUPPORTED, "mla_decode: only the FP8 per-token-scale row pool is built (dtype %d)",
                cache_dtype);
  if (B < 0 || num_heads < 1 || page_size < 16 || page_size % 16 || num_blocks < 1 || table_width < 0 ||
      table_stride < table_width || !(sm_scale > 0.0f))
    return fail(SNA_ERR_INVALID_ARGUMENT, "mla_decode: bad sizes (B %d, heads %d, page %d (a multiple of 16), blocks "
                "%lld, table %d/%lld)", B, num_heads, page_size, (long long)num_blocks, table_width,
                (long long)table_stride);
  if (!plan || plan->tile != 16 || plan->split_tiles < 1 || plan->n_work < 0)
    return fail(SNA_ERR_INVALID_ARGUMENT, "mla_decode: missing or foreign split plan");
  if (B == 0) return SNA_OK;
  if (!ql_nope || !q_pe || !cache || !row_scale || !block_table || !seq_lens || !compact_new || !out ||
      (plan->n_work > 0 && !workspace))
    return fail(SNA_ERR_INVALID_ARGUMENT, "mla_decode: null pointer");
  if (!aligned(ql_nope, 16) || !aligned(q_pe, 16) || !aligned(cache, 16) || !aligned(row_scale, 16))
    return fail(SNA_ERR_INVALID_ARGUMENT, "mla_decode: q, cache and row_scale must be 16-byte aligned");
  const int32_t groups = (num_heads + 15) / 16;
  const int64_t need = sna_decode_workspace_bytes(plan, num_heads, kLatent);
  if (plan->n_work > 0 && workspace_bytes < need)
    return fail(SNA_ERR_WORKSPACE, "mla_decode: workspace of %lld bytes, the plan needs %lld",
                (long long)workspace_bytes, (long long)need);
  float* ws = (float*)workspace;
  MlaArgs da{};
  da.ql = (const uint16_t*)ql_nope;
  da.qpe = (const uint16_t*)q_pe;
  da.cache = (const uint8_t*)cache;
  da.row_scale = row_scale;
  da.kv_scale = 1.0f;
  da.table = block_table;
  da.table_stride = table_stride;
  da.table_width = table_width;
  da.seq_lens = seq_lens;
  da.B = B;
  da.H = num_heads;
  da.P = page_size;
  da.num_blocks = num_blocks;
  da.sm_scale = sm_scale;
  da.split_tiles = plan->split_tiles;
  da.n_work = plan->n_work;
  da.ws_o = ws;
  da.ws_ml = ws ? ws + (int64_t)plan->n_work * num_heads * kLatent : nullptr;
  MlaCombineArgs ca{};
  ca.ql = da.ql;
  ca.qpe = da.qpe;
  ca.own = (const uint16_t*)compact_new;
  ca.new_slots = new_slots;
  ca.cache = (uint8_t*)cache;
  ca.row_scale = (float*)row_scale;
  ca.kv_scale = 1.0f;
  ca.seq_lens = seq_lens;
  ca.B = B;
  ca.H = num_heads;
  ca.P = page_size;
  ca.num_blocks = num_blocks;
  ca.sm_scale = sm_scale;
  ca.split_tiles = plan->split_tiles;
  ca.n_work = plan->n_work;
  ca.ws_o = da.ws_o;
  ca.ws_ml = da.ws_ml;
  ca.out = (uint16_t*)out;
  ca.lse_out = nullptr;
  hipStream_t s = (hipStream_t)stream;
  if (plan->n_work > 0)
    hipLaunchKernelGGL((mla_decode_kernel<ROWS576, 4>), dim3(plan->n_work, groups), dim3(256), 0, s, da);
  hipLaunchKernelGGL((mla_combine_kernel<ROWS576>), dim3(B, groups), dim3(256), 0, s, ca);
  return check_launch("mla_decode");
}

extern "C" int sna_mla_decode_sparse(const void* q_absorbed, const void* q_pe, const void* cache, float kv_scale,
                                     const int32_t* indices, int32_t n_indices, const int32_t* block_table,
                                     int64_t table_stride, int32_t table_width, const int32_t* positions,
                                     const void* own_rows, float sm_scale, void* ctx_out, float* lse_out, int32_t B,
                                     int32_t num_heads, int32_t page_size, int64_t num_blocks,
                                     const sna_split_plan* plan, void* workspace, int64_t workspace_bytes,
                                     void* stream) {
  ApiGuard guard;
  if (B < 0 || num_heads < 1 || n_indices < 0 || page_size < 1 || num_blocks < 1 || table_width < 0 ||
      table_stride < table_width || !(sm_scale > 0.0f) || !(kv_scale > 0.0f))
    return fail(SNA_ERR_INVALID_ARGUMENT, "mla_decode_sparse: bad sizes (B %d, heads %d, indices %d, page %d, blocks "
                "%lld, table %d/%lld, kv_scale %g)", B, num_heads, n_indices, page_size, (long long)num_blocks,
                table_width, (long long)table_stride, (double)kv_scale);
  if (!plan || plan->tile != 16 || plan->split_tiles < 1 || plan->n_work < 0)
    return fail(SNA_ERR_INVALID_ARGUMENT, "mla_decode_sparse: missing or foreign split plan");
  if (B == 0) return SNA_OK;
  if (!q_absorbed || !q_pe || !cache || !block_table || !positions || !own_rows || !ctx_out ||
      (n_indices > 0 && !indices) || (plan->n_work > 0 && !workspace))
    return fail(SNA_ERR_INVALID_ARGUMENT, "mla_decode_sparse: null pointer");
  if (!aligned(q_absorbed, 16) || !aligned(q_pe, 16) || !aligned(cache, 16))
    return fail(SNA_ERR_INVALID_ARGUMENT, "mla_decode_sparse: q and cache must be 16-byte aligned");
  const int32_t per = (n_indices + 15) / 16 == 0 ? 0 : ((n_indices + 15) / 16 + plan->split_tiles - 1) / plan->split_tiles;
  if ((int64_t)per * B > plan->n_work)
    return fail(SNA_ERR_INVALID_ARGUMENT, "mla_decode_sparse: the plan holds %d items, the index lists need %lld",
                plan->n_work, (long long)per * B);
  const int32_t groups = (num_heads + 15) / 16;
  const int64_t need = sna_decode_workspace_bytes(plan, num_heads, kLatent);
  if (plan->n_work > 0 && workspace_bytes < need)
    return fail(SNA_ERR_WORKSPACE, "mla_decode_sparse: workspace of %lld bytes, the plan needs %lld",
                (long long)workspace_bytes, (long long)need);
  float* ws = (float*)workspace;
  MlaArgs da{};
  da.ql = (const uint16_t*)q_absorbed;
  da.qpe = (const uint16_t*)q_pe;
  da.cache = (const uint8_t*)cache;
  da.row_scale = nullptr;
  da.kv_scale = kv_scale;
  da.table = block_table;
  da.table_stride = table_stride;
  da.table_width = table_width;
  da.indices = indices;
  da.n_indices = n_indices;
  da.positions = positions;
  da.B = B;
  da.H = num_heads;
  da.P = page_size;
  da.num_blocks = num_blocks;
  da.sm_scale = sm_scale;
  da.split_tiles = plan->split_tiles;
  da.n_work = plan->n_work;
  da.ws_o = ws;
  da.ws_ml = ws ? ws + (int64_t)plan->n_work * num_heads * kLatent : nullptr;
  MlaCombineArgs ca{};
  ca.ql = da.ql;
  ca.qpe = da.qpe;
  ca.own = (const uint16_t*)own_rows;
  ca.new_slots = nullptr;
  ca.kv_scale = kv_scale;
  ca.n_indices = n_indices;
  ca.B = B;
  ca.H = num_heads;
  ca.P = page_size;
  ca.num_blocks = num_blocks;
  ca.sm_scale = sm_scale;
  ca.split_tiles = plan->split_tiles;
  ca.n_work = plan->n_work;
  ca.ws_o = da.ws_o;
  ca.ws_ml = da.ws_ml;
  ca.out = (uint16_t*)ctx_out;
  ca.lse_out = lse_out;
  hipStream_t s = (hipStream_t)stream;
  if (per * B > 0)
    hipLaunchKernelGGL((mla_decode_kernel<ROWS640, 4>), dim3(per * B, groups), dim3(256), 0, s, da);
  hipLaunchKernelGGL((mla_combine_kernel<ROWS640>), dim3(B, groups), dim3(256), 0, s, ca);
  return check_launch("mla_decode_sparse");
}
