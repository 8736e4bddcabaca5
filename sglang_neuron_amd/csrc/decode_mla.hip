// Absorbed-MLA decode (paged, per-token FP8 scale) and DSA sparse decode (index lists over 640-byte packed rows):
// split-K online softmax with all 16 heads of a head group in one wave, MFMA for QK^T and PV. The workgroup of a
// row's first split also attends the row's own new token in-band (and, paged, stores it). A row with one split
// writes its final output; otherwise a combine pass merges the splits.
//
// Row formats:
//   ROWS576  [latent 512 | k_pe 64] e4m3fn, one fp32 dequantization scale per token slot (row_scale).
//   ROWS640  [k_pe 64 bf16 | latent 512 e4m3fn, permuted], one per-tensor kv_scale. Latent dim c = 256a + 128b + p
//            sits at latent byte 256a + 2p + b.
//
// Work: one workgroup of 4 waves per (row, split, 16-head group). The workgroup first resolves the row id of every
// key of its split into LDS (the block-table walk, or for DSA the index -> block -> row walk). Each wave then takes
// 16-key tiles round-robin through a ring of 3 LDS slots, filled by global->LDS DMA: two tiles are in flight while
// it computes a third, and the in-flight bytes cost no registers.
//
// Lane roles (lane = 16 * g4 + li), 16-key tiles:
//   QK   S^T[key, head] = K[key, :] . Q[head, :]   v_mfma_f32_16x16x32_bf16, 18 steps over the 576 dims. Lane
//        (g4, li) feeds 144 (ROWS576) or 160 (ROWS640) bytes of key li's row, loaded straight from HBM, and head li's
//        query elements under the same K-index map. The query operand lives in LDS in lane order.
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
constexpr int kLdsRow = 528;        // latent bytes of one key row in LDS, padded so rows 4 apart hit other banks
constexpr int kMlaRingDepth = 3;    // LDS tile slots per wave
constexpr float kMlaRescaleSlack = 8.0f;

struct MlaArgs {
  const uint16_t* ql;    // [B, H, 512]
  const uint16_t* qpe;   // [B, H, 64]
  uint8_t* cache;        // rows
  float* row_scale;      // ROWS576
  float kv_scale;        // ROWS640
  const int32_t* table;
  int64_t table_stride;
  int32_t table_width;
  const int32_t* seq_lens;   // paged
  const int32_t* indices;    // sparse [B, n_indices]
  int32_t n_indices;
  const int32_t* positions;  // sparse [B]
  const uint16_t* own;       // [B, 576] bf16: ROWS576 [latent | rope], ROWS640 [rope | latent]
  const int64_t* new_slots;  // paged: store the own row there (NULL: no store)
  int32_t B, H, P;
  int64_t num_blocks;
  float sm_scale;
  int32_t split_tiles, n_work, max_splits;
  float* ws_o;   // [B, max_splits, H, 512]  unnormalized partials, latent-byte order
  float* ws_ml;  // [B, max_splits, H, 2]
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

// Latent byte offset of chunk c of lane group g4, or -1 for a rope chunk.
template <int FMT>
__device__ __forceinline__ int chunk_latent(int g4, int c) {
  if constexpr (FMT == ROWS576) {
    const int off = 144 * g4 + 16 * c;
    return off < kLatent ? off : -1;
  } else {
    return c < 2 ? -1 : 128 * g4 + 16 * (c - 2);
  }
}

// The query element pair-block of step s, lane group g4 for head row qlp/qpp (8 bf16, packed).
template <int FMT>
__device__ __forceinline__ uint4 query_chunk(const uint16_t* qlp, const uint16_t* qpp, int g4, int s) {
  if constexpr (FMT == ROWS576) {
    const int dim = 144 * g4 + 8 * s;  // natural order: latent then rope
    return dim < kLatent ? ld16(qlp + dim) : ld16(qpp + (dim - kLatent));
  } else {
    if (s < 2) return ld16(qpp + 16 * g4 + 8 * s);
    uint32_t e[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = qlp[latent_dim_of_byte(128 * g4 + 8 * (s - 2) + i)];
    return make_uint4(e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16), e[6] | (e[7] << 16));
  }
}

// The own row of sequence b, dequantized in natural order [latent 512 | rope 64] into sm_row, stored into the
// pool when paged and st is set. Every thread of the workgroup calls it. ROWS576 quantizes with the row's own
// per-token scale, ROWS640 with kv_scale and the row's bf16 rope.
template <int FMT, int NT>
__device__ void own_row_dequant(const MlaArgs& a, int b, bool st, float* sm_row, float* sm_red) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint16_t* own = a.own + (int64_t)b * 576;
  if constexpr (FMT == ROWS576) {
    float m = 0.0f;
    for (int i = tid; i < 576; i += NT) m = fmaxf(m, fabsf(bf16_bits_to_f32(own[i])));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if (lane == 0) sm_red[wave] = m;
    __syncthreads();
    float mm = sm_red[0];
    for (int w = 1; w < NT / 64; ++w) mm = fmaxf(mm, sm_red[w]);
    const float s = scale_from_absmax(mm);
    int64_t slot = -1;
    if (st && a.new_slots) slot = redirect_slot(a.new_slots[b], a.num_blocks * a.P);
    for (int i = tid; i < 576; i += NT) {
      const uint32_t qb = quantize_e4m3fn(own[i], s);
      sm_row[i] = e4m3fn_to_f32(qb) * s;
      if (slot >= 0) a.cache[slot * 576 + i] = (uint8_t)qb;
    }
    if (slot >= 0 && tid == 0) a.row_scale[slot] = s;
  } else {
    for (int i = tid; i < 576; i += NT) {
      const uint32_t bits = own[i];
      if (i < kRope)
        sm_row[kLatent + i] = bf16_bits_to_f32(f32_to_bf16_bits(bf16_bits_to_f32(bits) / a.kv_scale)) * a.kv_scale;
      else
        sm_row[i - kRope] = e4m3fn_to_f32(quantize_e4m3fn(bits, a.kv_scale)) * a.kv_scale;
    }
  }
  __syncthreads();
}

// Score of the own row for heads [16 hg, 16 hg + nh), log2 domain, into sm_sn.
template <int NT>
__device__ void own_row_scores(const MlaArgs& a, int b, int hg, int nh, const float* sm_row, float* sm_sn) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int j = wave; j < nh; j += NT / 64) {
    const int32_t h = 16 * hg + j;
    const uint16_t* qlp = a.ql + ((int64_t)b * a.H + h) * kLatent;
    const uint16_t* qpp = a.qpe + ((int64_t)b * a.H + h) * kRope;
    float s = 0.0f;
    for (int d = lane; d < kLatent; d += 64) s += bf16_bits_to_f32(qlp[d]) * sm_row[d];
    s += bf16_bits_to_f32(qpp[lane]) * sm_row[kLatent + lane];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if (lane == 0) sm_sn[j] = s * a.sm_scale * kLog2e;
  }
  __syncthreads();
}

// Tile geometry in LDS. A tile is 16 rows of CH 16-byte chunks, loaded by NDMA wave-wide global->LDS DMAs (lane i of
// DMA j fills LDS chunk 64 j + i). Logical chunk c of row r sits at LDS chunk r * CH + (c + r / ROT) % CH: the per-row
// rotation spreads the rows a QK read touches over all LDS banks. Each lane's global address absorbs the rotation, so
// it costs nothing at load time.
template <int FMT>
struct TileGeo {
  static constexpr int CH = FMT == ROWS576 ? 36 : 40;
  static constexpr int NDMA = CH * 16 / 64;  // 9 or 10
  static constexpr int SLOT = NDMA * 1024;   // bytes of one ring slot
  static constexpr int ROT = FMT == ROWS576 ? 4 : 2;
  __device__ static int lds_chunk(int r, int c) {
    int x = c + r / ROT;
    x = x >= CH ? x - CH : x;
    return r * CH + x;
  }
};

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <int FMT, int WAVES, bool FINAL>
__global__ __launch_bounds__(64 * WAVES) void mla_decode_kernel(MlaArgs a) {
  using Geo = TileGeo<FMT>;
  constexpr int CH = Geo::CH;
  constexpr int NDMA = Geo::NDMA;
  constexpr int SLOT = Geo::SLOT;
  constexpr int ROWB = RowFmt<FMT>::kRowBytes;
  constexpr bool SPARSE = FMT == ROWS640;
  constexpr int NT = 64 * WAVES;
  constexpr int DEPTH = kMlaRingDepth;
  // VMEM operations one tile issues: its DMAs, plus the per-token scale load of the paged format
  constexpr int PER_TILE = NDMA + (SPARSE ? 0 : 1);
  typedef __attribute__((address_space(3))) void lds_void;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int g4 = lane >> 4;
  const int li = lane & 15;
  const int hg = blockIdx.y;  // 16-head group
  const int nh = min(16, a.H - 16 * hg);

  // LDS: the query operand, the split's row ids, and each wave's ring of DEPTH tile slots. After the tile loop the
  // ring's space holds the merge buffers.
  __shared__ uint4 sm_q[18][64];
  __shared__ int32_t sm_rowid[kMlaMaxSplitKeys];
  __shared__ __attribute__((aligned(1024))) uint8_t sm_ring[WAVES][DEPTH][SLOT];
  __shared__ float sm_m[WAVES][16];
  __shared__ float sm_l[WAVES][16];
  __shared__ float sm_row[576];
  __shared__ float sm_sn[16];
  __shared__ float sm_red[WAVES];
  static_assert(sizeof(float) * 16 * (kLatent + 4) <= sizeof(sm_ring), "the merge buffer lives in the ring");
  float(*sm_o)[kLatent + 4] = reinterpret_cast<float(*)[kLatent + 4]>(&sm_ring[0][0][0]);

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
    b = __builtin_amdgcn_readfirstlane(b);
    split = __builtin_amdgcn_readfirstlane(split);
  }
  if (b < 0) return;

  const int32_t khi = SPARSE ? a.n_indices : ld_const(a.seq_lens + b) - 1;
  const int32_t t_first = split * a.split_tiles;
  const int32_t t_last = min(t_first + a.split_tiles, (khi + 15) / 16);
  const int32_t kbase = t_first * 16;
  const int32_t nkeys = (t_last - t_first) * 16;

  // ---- the query operand into LDS, and every key's row id ----
  for (int e = tid; e < 18 * 64; e += NT) {
    const int s = e >> 6, ln = e & 63;
    const int32_t h = 16 * hg + (ln & 15);
    uint4 w = make_uint4(0, 0, 0, 0);
    if (h < a.H) {
      const uint16_t* qlp = a.ql + ((int64_t)b * a.H + h) * kLatent;
      const uint16_t* qpp = a.qpe + ((int64_t)b * a.H + h) * kRope;
      w = query_chunk<FMT>(qlp, qpp, ln >> 4, s);
    }
    sm_q[s][ln] = w;
  }
  const int32_t* trow = a.table + (int64_t)b * a.table_stride;
  const int64_t n_rows = a.num_blocks * a.P;
  int32_t qpos = 0;
  if constexpr (SPARSE) qpos = a.positions[b];
  for (int k = tid; k < nkeys; k += NT) {
    const int32_t key = kbase + k;
    int32_t row = -1;
    if constexpr (SPARSE) {
      const int32_t pos = key < khi ? a.indices[(int64_t)b * a.n_indices + key] : -1;
      if (pos >= 0 && pos <= qpos) {
        const int32_t blk = pos / a.P;
        if (blk < a.table_width) {
          const int32_t e = trow[blk];
          if (e >= 0 && (int64_t)e < a.num_blocks) {
            const int64_t r = (int64_t)e * a.P + pos % a.P;
            if (r < n_rows) row = (int32_t)r;
          }
        }
      }
    } else {
      if (key < khi) {
        const int32_t col = key / a.P;
        const int32_t e = col < a.table_width ? trow[col] : -1;
        if (e >= 0 && (int64_t)e < a.num_blocks) row = e * a.P + key % a.P;
      }
    }
    sm_rowid[k] = row;
  }
  __syncthreads();
  // the query operand in registers for the whole tile loop
  uint32_t qv[18][4];
#pragma unroll
  for (int s = 0; s < 18; ++s) {
    const uint4 w = sm_q[s][lane];
    qv[s][0] = w.x;
    qv[s][1] = w.y;
    qv[s][2] = w.z;
    qv[s][3] = w.w;
  }

  // Each lane's (row, chunk) for every DMA of a tile: fixed by the layout.
  int dma_row[NDMA], dma_off[NDMA];
#pragma unroll
  for (int j = 0; j < NDMA; ++j) {
    const int o = 64 * j + lane;
    const int r = o / CH, sl = o % CH;
    int c = sl - r / Geo::ROT;
    c = c < 0 ? c + CH : c;
    dma_row[j] = r;
    dma_off[j] = 16 * c;
  }

  float kscale_ring[DEPTH][4];
  // Issue the loads of tile `tile` into ring slot `slot`: NDMA DMAs, and the per-token scales into registers.
  auto issue = [&](int slot, int32_t tile, float (&ks)[4]) {
    const int32_t k0 = tile * 16 - kbase;
    uint8_t* dst = sm_ring[wave][slot];
#pragma unroll
    for (int j = 0; j < NDMA; ++j) {
      const int32_t row = sm_rowid[k0 + dma_row[j]];
      const uint8_t* src = a.cache + (int64_t)(row >= 0 ? row : 0) * ROWB + dma_off[j];
      __builtin_amdgcn_global_load_lds((const void*)src, (lds_void*)(dst + 1024 * j), 16, 0, 0);
    }
    if constexpr (!SPARSE) {
      // per-token scales of keys 4 g4 .. 4 g4 + 3: consecutive slots of one page
      const int32_t srow = sm_rowid[k0 + 4 * g4];
      const float4 s4 = *reinterpret_cast<const float4*>(a.row_scale + (srow >= 0 ? srow : 0));
      ks[0] = s4.x;
      ks[1] = s4.y;
      ks[2] = s4.z;
      ks[3] = s4.w;
    }
  };

  const float base_scale = a.sm_scale * kLog2e * (SPARSE ? a.kv_scale : 1.0f);
  float m_ref = kNegBig;
  float l_run = 0.0f;
  f32x4_t acc[8][4];
#pragma unroll
  for (int q = 0; q < 8; ++q)
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[q][r] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int slot, int32_t tile, const float (&ks)[4]) {
    const uint8_t* T = sm_ring[wave][slot];
    const int32_t k0 = tile * 16 - kbase;
    // validity of the tile's keys (bit k: key k)
    const uint32_t vmask = (uint32_t)(__ballot(sm_rowid[k0 + li] >= 0) & 0xffffull);
    // S^T = K Q^T from the slot: lane (g4, li) reads its chunks of row li. Three accumulators keep three
    // independent MFMA chains in flight; they are summed at the end.
    f32x4_t scp[3] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int s = 0; s < 18; s += 2) {
      // the two MFMA steps s, s + 1 share one 16-byte chunk
      f32x4_t& sc = scp[(s / 2) % 3];
      if constexpr (FMT == ROWS640) {
        if (s == 0) {
          // steps 0 and 1: the bf16 rope, one chunk each
          const uint4 w0 = *reinterpret_cast<const uint4*>(T + 16 * Geo::lds_chunk(li, 2 * g4));
          const uint4 w1 = *reinterpret_cast<const uint4*>(T + 16 * Geo::lds_chunk(li, 2 * g4 + 1));
          const uint32_t a0[4] = {w0.x, w0.y, w0.z, w0.w}, a1[4] = {w1.x, w1.y, w1.z, w1.w};
          sc = mfma_16x16x32_bf16(a0, qv[0], sc);
          sc = mfma_16x16x32_bf16(a1, qv[1], sc);
          continue;
        }
      }
      const int c = FMT == ROWS576 ? 9 * g4 + s / 2 : 8 + 8 * g4 + (s - 2) / 2;
      const uint4 w = *reinterpret_cast<const uint4*>(T + 16 * Geo::lds_chunk(li, c));
      uint32_t op0[4], op1[4];
      fp8x4_to_bf16x4(w.x, op0[0], op0[1]);
      fp8x4_to_bf16x4(w.y, op0[2], op0[3]);
      fp8x4_to_bf16x4(w.z, op1[0], op1[1]);
      fp8x4_to_bf16x4(w.w, op1[2], op1[3]);
      sc = mfma_16x16x32_bf16(op0, qv[s], sc);
      sc = mfma_16x16x32_bf16(op1, qv[s + 1], sc);
    }
    const f32x4_t sc = scp[0] + scp[1] + scp[2];
    // mask, online softmax with a lazily moved reference maximum
    float x[4];
    float tmax = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool ok = (vmask >> (4 * g4 + r)) & 1u;
      const float kscl = SPARSE ? 1.0f : ks[r];
      x[r] = ok ? sc[r] * base_scale * kscl : -INFINITY;
      tmax = fmaxf(tmax, x[r]);
    }
    tmax = max_across_groups(tmax);
    const bool bump = tmax > m_ref + kMlaRescaleSlack;
    if (__any(bump)) {
      const float m_new = bump ? tmax : m_ref;
      const float alpha = __builtin_amdgcn_exp2f(m_ref - m_new);
      m_ref = m_new;
      l_run *= alpha;
#pragma unroll
      for (int q = 0; q < 8; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[q][r] *= alpha;
    }
    float pv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool ok = (vmask >> (4 * g4 + r)) & 1u;
      const float p = __builtin_amdgcn_exp2f(x[r] - m_ref);
      l_run += p;
      // V is dequantized through P: p' = p * scale(key); a masked key has p = 0
      pv[r] = ok ? p * (SPARSE ? 1.0f : ks[r]) : 0.0f;
    }
    const uint32_t pop[2] = {pack_bf16x2(pv[0], pv[1]), pack_bf16x2(pv[2], pv[3])};
    const bool full = vmask == 0xffffu;
    // O^T += V^T P^T over 32 d-tiles: lane (g4, i) reads latent dword 64 q + 4 i of rows 4 g4 .. 4 g4 + 3
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      uint32_t w[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 4 * g4 + e;
        const int rb = (SPARSE ? 128 : 0) + 64 * q + 4 * li;  // the dword's byte within the row
        w[e] = *reinterpret_cast<const uint32_t*>(T + 16 * Geo::lds_chunk(r, rb >> 4) + (rb & 15));
        // a masked key's bytes may be anything (a stale NaN would survive p = 0): zero them
        if (!full) w[e] = ((vmask >> r) & 1u) ? w[e] : 0u;
      }
      uint32_t xr[4];
      transpose4x4_bytes(w, xr);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        uint32_t op[2];
        fp8x4_to_bf16x4(xr[r], op[0], op[1]);
        acc[q][r] = mfma_16x16x16_bf16(op, pop, acc[q][r]);
      }
    }
  };

  // ---- the tile loop: DEPTH ring slots per wave, DEPTH - 1 tiles' loads in flight while one computes ----
  {
    const int32_t t0 = t_first + wave;
#pragma unroll
    for (int i = 0; i < DEPTH - 1; ++i)
      if (t0 + i * WAVES < t_last) issue(i, t0 + i * WAVES, kscale_ring[i]);
    for (int32_t base = 0;; base += DEPTH) {
      bool done = false;
#pragma unroll
      for (int k = 0; k < DEPTH; ++k) {
        const int32_t cur = t0 + (base + k) * WAVES;
        if (cur >= t_last) {
          done = true;
          break;
        }
        // issue the tile DEPTH - 1 ahead, then wait until this tile's loads have landed: the ones issued after it
        // (up to DEPTH - 1 tiles' worth) may stay in flight
        const int32_t nxt = cur + (DEPTH - 1) * WAVES;
        if (nxt < t_last) {
          issue((k + DEPTH - 1) % DEPTH, nxt, kscale_ring[(k + DEPTH - 1) % DEPTH]);
          wait_vmcnt<(DEPTH - 1) * PER_TILE>();
        } else if (nxt - WAVES < t_last && DEPTH > 2) {
          wait_vmcnt<(DEPTH - 2) * PER_TILE>();
        } else {
          wait_vmcnt<0>();
        }
        compute(k, cur, kscale_ring[k]);
      }
      if (done) break;
    }
    wait_vmcnt<0>();
  }

  // ---- the own row, attended in-band by the row's first split (paged: and stored, by head group 0) ----
  const bool own = split == 0;  // uniform
  __syncthreads();  // every wave is done with the ring before its space becomes the merge buffer
  if (own) {
    own_row_dequant<FMT, NT>(a, b, hg == 0, sm_row, sm_red);
    own_row_scores<NT>(a, b, hg, nh, sm_row, sm_sn);
  }

  // ---- merge: a common maximum per head, then the waves' rescaled accumulators summed through LDS ----
  const float l_tot = sum_across_groups(l_run);
  if (g4 == 0) {
    sm_m[wave][li] = m_ref;
    sm_l[wave][li] = l_tot;
  }
  __syncthreads();
  float M = own ? sm_sn[li] : -INFINITY;
#pragma unroll
  for (int w = 0; w < WAVES; ++w) M = fmaxf(M, sm_m[w][li]);
  const float f = __builtin_amdgcn_exp2f(m_ref - M);
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
  const float oscale = SPARSE ? a.kv_scale : 1.0f;
  const int32_t S = a.max_splits;
  for (int idx = tid; idx < nh * kLatent; idx += NT) {
    const int j = idx / kLatent, c = idx % kLatent;  // c: the latent dim written (FINAL), or byte (partial)
    const int32_t h = 16 * hg + j;
    float Mj = own ? sm_sn[j] : -INFINITY;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) Mj = fmaxf(Mj, sm_m[w][j]);
    float l = 0.0f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) l += __builtin_amdgcn_exp2f(sm_m[w][j] - Mj) * sm_l[w][j];
    const float e_own = own ? __builtin_amdgcn_exp2f(sm_sn[j] - Mj) : 0.0f;
    l += e_own;
    if constexpr (FINAL) {
      const int beta = SPARSE ? latent_byte_of_dim(c) : c;
      float o = sm_o[j][beta] * oscale;
      if (own) o += e_own * sm_row[c];
      a.out[((int64_t)b * a.H + h) * kLatent + c] = (uint16_t)f32_to_bf16_bits(o / l);
      if (a.lse_out && c == 0) a.lse_out[(int64_t)b * a.H + h] = (Mj + __log2f(l)) * 0.6931471805599453f;
    } else {
      const int beta = c;
      float o = sm_o[j][beta] * oscale;
      if (own) o += e_own * sm_row[SPARSE ? latent_dim_of_byte(beta) : beta];
      const int64_t row = ((int64_t)b * S + split) * a.H + h;
      a.ws_o[row * kLatent + beta] = o;
      if (beta == 0) {
        a.ws_ml[row * 2] = Mj;
        a.ws_ml[row * 2 + 1] = l;
      }
    }
  }
}

// Merge of a row's splits per (row, head): out = sum_s e_s o_s / sum_s e_s l_s, lse = M + log(sum), with
// e_s = exp2(m_s - M) formed once per head in LDS.
template <int FMT>
__global__ __launch_bounds__(128) void mla_combine_kernel(MlaArgs a) {
  constexpr bool SPARSE = FMT == ROWS640;
  const int b = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
  const int32_t n = min(SPARSE ? splits_of<16>(a.n_indices + 1, 0, a.split_tiles)
                               : splits_of<16>(ld_const(a.seq_lens + b), 0, a.split_tiles),
                        a.max_splits);
  __shared__ float sm_w[kMaxSplits];
  __shared__ float sm_l[kMaxSplits];
  __shared__ float sm_inv, sm_lse;
  const int64_t row0 = (int64_t)b * a.max_splits * a.H + h;
  for (int s = tid; s < n; s += blockDim.x) {
    const float2 ml = *reinterpret_cast<const float2*>(a.ws_ml + (row0 + (int64_t)s * a.H) * 2);
    sm_w[s] = ml.x;
    sm_l[s] = ml.y;
  }
  __syncthreads();
  if (tid == 0) {
    float M = -INFINITY;
    for (int32_t s = 0; s < n; ++s) M = fmaxf(M, sm_w[s]);
    float den = 0.0f;
    for (int32_t s = 0; s < n; ++s) {
      const float w = __builtin_amdgcn_exp2f(sm_w[s] - M);
      sm_w[s] = w;
      den += w * sm_l[s];
    }
    sm_inv = 1.0f / den;
    sm_lse = (M + __log2f(den)) * 0.6931471805599453f;
  }
  __syncthreads();
  const float* ob = a.ws_o + row0 * kLatent;
  for (int c = tid; c < kLatent; c += blockDim.x) {
    const int beta = SPARSE ? latent_byte_of_dim(c) : c;
    float num = 0.0f;
#pragma unroll 8
    for (int32_t s = 0; s < n; ++s) num += sm_w[s] * ob[(int64_t)s * a.H * kLatent + beta];
    a.out[((int64_t)b * a.H + h) * kLatent + c] = (uint16_t)f32_to_bf16_bits(num * sm_inv);
  }
  if (a.lse_out && tid == 0) a.lse_out[(int64_t)b * a.H + h] = sm_lse;
}

// A row with no prior key (paged seq_len 1, or an empty index list): the output is its own row's latent.
template <int FMT>
__global__ __launch_bounds__(256) void mla_lone_row_kernel(MlaArgs a) {
  constexpr bool SPARSE = FMT == ROWS640;
  const int b = blockIdx.x, hg = blockIdx.y;
  const int32_t n = SPARSE ? splits_of<16>(a.n_indices + 1, 0, a.split_tiles)
                           : splits_of<16>(a.seq_lens[b], 0, a.split_tiles);
  if (n > 0) return;
  __shared__ float sm_row[576];
  __shared__ float sm_sn[16];
  __shared__ float sm_red[4];
  const int nh = min(16, a.H - 16 * hg);
  own_row_dequant<FMT, 256>(a, b, hg == 0, sm_row, sm_red);
  own_row_scores<256>(a, b, hg, nh, sm_row, sm_sn);
  for (int idx = threadIdx.x; idx < nh * kLatent; idx += 256) {
    const int j = idx / kLatent, c = idx % kLatent;
    const int32_t h = 16 * hg + j;
    a.out[((int64_t)b * a.H + h) * kLatent + c] = (uint16_t)f32_to_bf16_bits(sm_row[c]);
    if (a.lse_out && c == 0) a.lse_out[(int64_t)b * a.H + h] = sm_sn[j] * 0.6931471805599453f;
  }
}

template <int FMT>
static void launch_mla(const MlaArgs& a, int32_t groups, int32_t grid_x, bool any_lone, hipStream_t s) {
  timing_mark(0, s);
  if (grid_x > 0) {
    if (a.max_splits <= 1)
      hipLaunchKernelGGL((mla_decode_kernel<FMT, 4, true>), dim3(grid_x, groups), dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((mla_decode_kernel<FMT, 4, false>), dim3(grid_x, groups), dim3(256), 0, s, a);
  }
  timing_mark(1, s);
  if (a.max_splits > 1) hipLaunchKernelGGL((mla_combine_kernel<FMT>), dim3(a.B, a.H), dim3(128), 0, s, a);
  if (any_lone) hipLaunchKernelGGL((mla_lone_row_kernel<FMT>), dim3(a.B, groups), dim3(256), 0, s, a);
  timing_mark(2, s);
}

static int check_plan(const sna_split_plan* plan, int32_t B, const char* what) {
  if (!plan || plan->tile != 16 || plan->split_tiles < 1 || plan->n_work < 0 || plan->max_splits < 0 ||
      plan->batch != B)
    return fail(SNA_ERR_INVALID_ARGUMENT, "%s: missing or foreign split plan (made for %d rows)", what,
                plan ? plan->batch : -1);
  if (plan->split_tiles * 16 > kMlaMaxSplitKeys)
    return fail(SNA_ERR_INVALID_ARGUMENT, "%s: a split of %d keys exceeds the kernel's %d", what,
                plan->split_tiles * 16, kMlaMaxSplitKeys);
  return SNA_OK;
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
      table_stride < table_width || !(sm_scale > 0.0f) || num_blocks * page_size > INT32_MAX)
    return fail(SNA_ERR_INVALID_ARGUMENT, "mla_decode: bad sizes (B %d, heads %d, page %d (a multiple of 16), blocks "
                "%lld, table %d/%lld)", B, num_heads, page_size, (long long)num_blocks, table_width,
                (long long)table_stride);
  if (int rc = check_plan(plan, B, "mla_decode")) return rc;
  if (B == 0) return SNA_OK;
  const int64_t need = sna_decode_workspace_bytes(plan, num_heads, kLatent);
  if (!ql_nope || !q_pe || !cache || !row_scale || !block_table || !seq_lens || !compact_new || !out ||
      (need > 0 && !workspace))
    return fail(SNA_ERR_INVALID_ARGUMENT, "mla_decode: null pointer");
  if (!aligned(ql_nope, 16) || !aligned(q_pe, 16) || !aligned(cache, 16) || !aligned(row_scale, 16))
    return fail(SNA_ERR_INVALID_ARGUMENT, "mla_decode: q, cache and row_scale must be 16-byte aligned");
  if (workspace_bytes < need)
    return fail(SNA_ERR_WORKSPACE, "mla_decode: workspace of %lld bytes, the plan needs %lld",
                (long long)workspace_bytes, (long long)need);
  const int32_t groups = (num_heads + 15) / 16;
  float* ws = (float*)workspace;
  MlaArgs a{};
  a.ql = (const uint16_t*)ql_nope;
  a.qpe = (const uint16_t*)q_pe;
  a.cache = (uint8_t*)cache;
  a.row_scale = (float*)row_scale;
  a.kv_scale = 1.0f;
  a.table = block_table;
  a.table_stride = table_stride;
  a.table_width = table_width;
  a.seq_lens = seq_lens;
  a.own = (const uint16_t*)compact_new;
  a.new_slots = new_slots;
  a.B = B;
  a.H = num_heads;
  a.P = page_size;
  a.num_blocks = num_blocks;
  a.sm_scale = sm_scale;
  a.split_tiles = plan->split_tiles;
  a.n_work = plan->n_work;
  a.max_splits = plan->max_splits;
  a.ws_o = need > 0 ? ws : nullptr;
  a.ws_ml = need > 0 ? ws + (int64_t)B * plan->max_splits * num_heads * kLatent : nullptr;
  a.out = (uint16_t*)out;
  a.lse_out = nullptr;
  launch_mla<ROWS576>(a, groups, plan->n_work, plan->empty_rows != 0, (hipStream_t)stream);
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
      table_stride < table_width || !(sm_scale > 0.0f) || !(kv_scale > 0.0f) || num_blocks * page_size > INT32_MAX)
    return fail(SNA_ERR_INVALID_ARGUMENT, "mla_decode_sparse: bad sizes (B %d, heads %d, indices %d, page %d, blocks "
                "%lld, table %d/%lld, kv_scale %g)", B, num_heads, n_indices, page_size, (long long)num_blocks,
                table_width, (long long)table_stride, (double)kv_scale);
  if (int rc = check_plan(plan, B, "mla_decode_sparse")) return rc;
  if (B == 0) return SNA_OK;
  const int64_t need = sna_decode_workspace_bytes(plan, num_heads, kLatent);
  if (!q_absorbed || !q_pe || !cache || !block_table || !positions || !own_rows || !ctx_out ||
      (n_indices > 0 && !indices) || (need > 0 && !workspace))
    return fail(SNA_ERR_INVALID_ARGUMENT, "mla_decode_sparse: null pointer");
  if (!aligned(q_absorbed, 16) || !aligned(q_pe, 16) || !aligned(cache, 16))
    return fail(SNA_ERR_INVALID_ARGUMENT, "mla_decode_sparse: q and cache must be 16-byte aligned");
  const int32_t tiles = (n_indices + 15) / 16;
  const int32_t per = tiles == 0 ? 0 : (tiles + plan->split_tiles - 1) / plan->split_tiles;
  if (per > plan->max_splits || (int64_t)per * B > plan->n_work)
    return fail(SNA_ERR_INVALID_ARGUMENT, "mla_decode_sparse: the plan holds %d splits per row, the index lists need "
                "%d", plan->max_splits, per);
  if (workspace_bytes < need)
    return fail(SNA_ERR_WORKSPACE, "mla_decode_sparse: workspace of %lld bytes, the plan needs %lld",
                (long long)workspace_bytes, (long long)need);
  const int32_t groups = (num_heads + 15) / 16;
  float* ws = (float*)workspace;
  MlaArgs a{};
  a.ql = (const uint16_t*)q_absorbed;
  a.qpe = (const uint16_t*)q_pe;
  a.cache = (uint8_t*)cache;
  a.row_scale = nullptr;
  a.kv_scale = kv_scale;
  a.table = block_table;
  a.table_stride = table_stride;
  a.table_width = table_width;
  a.indices = indices;
  a.n_indices = n_indices;
  a.positions = positions;
  a.own = (const uint16_t*)own_rows;
  a.new_slots = nullptr;
  a.B = B;
  a.H = num_heads;
  a.P = page_size;
  a.num_blocks = num_blocks;
  a.sm_scale = sm_scale;
  a.split_tiles = plan->split_tiles;
  a.n_work = plan->n_work;
  a.max_splits = plan->max_splits;
  a.ws_o = need > 0 ? ws : nullptr;
  a.ws_ml = need > 0 ? ws + (int64_t)B * plan->max_splits * num_heads * kLatent : nullptr;
  a.out = (uint16_t*)ctx_out;
  a.lse_out = lse_out;
  launch_mla<ROWS640>(a, groups, per * B, per == 0, (hipStream_t)stream);
  return check_launch("mla_decode_sparse");
}
