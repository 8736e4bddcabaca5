// Absorbed-MLA decode (paged, per-token FP8 scale) and DSA sparse decode (index lists over 640-byte packed rows):
// split-K online softmax with all 16 heads of a head group in one wave, MFMA for QK^T and PV. The workgroup of a
// row's last split (paged; sparse: its first) also attends the row's own new token in-band (and, paged, stores it).
// A row with one split writes its final output; otherwise a combine pass merges the splits.
//
// Row formats:
//   ROWS576  [latent 512 | k_pe 64] e4m3fn, one fp32 dequantization scale per token slot (row_scale).
//   ROWS640  [k_pe 64 bf16 | latent 512 e4m3fn, permuted], one per-tensor kv_scale. Latent dim c = 256a + 128b + p
//            sits at latent byte 256a + 2p + b.
//
// Work: one workgroup of 4 waves per (row, split, 16-head group). Each wave takes the split's 16-key tiles
// round-robin through its own ring of LDS slots, filled by global->LDS DMA, so the in-flight bytes cost no
// registers. Paged: a tile is 16 consecutive slots of one page (the page size is a multiple of 16), one contiguous
// 9 KB run of HBM; the split's block-table entries sit in two VGPRs and a tile's page is a readlane. Sparse: the
// workgroup first resolves every index of its split to a row id in LDS (index -> block -> row). The own row is
// quantized as the store quantizes it and attended as a one-key tile by one wave of the row's last split (paged) or
// first split (sparse).
//
// Lane roles (lane = 16 * g4 + li), 16-key tiles; slot i of a tile (a row of S^T, a K index of PV) holds key
// key_of(i): the even keys in slots 0 .. 7, the odd ones in 8 .. 15.
//   QK   S^T[slot, head] = K[key, :] . Q[head, :]   v_mfma_f32_16x16x32_bf16, 18 steps over the 576 dims. In step
//        pair k lane (g4, li) feeds the 16 bytes of chunk 4 k + g4 of key key_of(li)'s row (ROWS640: the rope chunks
//        4 s + g4 first, then the latent chunks 8 + 4 (k - 1) + g4), and head li's query elements of the same dims
//        (from LDS).
//   PV   O^T[latent byte, head] = V^T[byte, slots] . P^T[slots, head]   v_mfma_f32_16x16x16_bf16, K = the 16 slots,
//        lane (g4, *) supplying slots 4 g4 .. 4 g4 + 3, the S^T rows it holds. One ds_read_b64_tr_b8 per 32 latent
//        bytes hands lane (g4, j) bytes 32 s + j and 32 s + 16 + j of those 4 slots' keys: d-tiles 2 s and 2 s + 1.
//   acc  lane (g4, j) accumulates head j at latent bytes 64 q + 16 r + 4 g4 + r'  (acc[q][r][r'], q < 8, r, r' < 4).
#include "sna_device.h"
#include "sna_host.h"

namespace sna {

enum { ROWS576 = 0, ROWS640 = 1 };

constexpr int kLatent = 512;
constexpr int kRope = 64;
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
  int32_t work_n;                   // entries of work (0: locate items from seq_lens)
  uint32_t work[SNA_MAX_WORK_MAP];  // item -> row << 6 | split, from the plan
  float* ws_o;   // [B, max_splits, H, 512]  unnormalized partials, latent-dim order
  float* ws_ml;  // [B, max_splits, H, 2]
  uint16_t* out;
  float* lse_out;
};

// The key in slot i of a tile. In a PV read, lanes 0 .. 31 then touch the 8 even rows and lanes 32 .. 63 the 8 odd
// ones; with the row strides below, 8 even rows fall in 8 distinct 8-bank blocks.
__device__ __forceinline__ int key_of(int i) { return 2 * (i & 7) + (i >> 3); }

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

// Tile geometry in LDS. A tile is 16 key rows; chunk c (16 bytes) of row r sits at LDS chunk r * STRIDE + c, with
// STRIDE = CHUNKS + 1: the pad chunk puts rows 1 apart 20 (ROWS576) or 36 (ROWS640) banks apart and rows 4 apart 16
// banks apart, so the QK reads (16 rows, one 16-byte chunk each) and the PV reads (4 rows x 64 bytes per lane group)
// are free of bank conflicts, and every LDS address is a per-lane base plus a constant. NDMA wave-wide DMAs fill a
// slot: lane i of DMA j fills LDS chunk 64 j + i. A pad chunk loads a duplicate of its row's last chunk; the lanes of
// the last DMA past the tile are switched off. ROWS576 tiles bring their 16 per-token scales along in one more DMA.
template <int FMT>
struct TileGeo {
  static constexpr int CHUNKS = FMT == ROWS576 ? 36 : 40;
  static constexpr int STRIDE = CHUNKS + 1;
  static constexpr int RS = 16 * STRIDE;                        // LDS row stride, bytes
  static constexpr int NDMA = (16 * STRIDE + 63) / 64;          // 10 or 11
  static constexpr int TAIL = 16 * STRIDE - 64 * (NDMA - 1);    // active lanes of the last DMA
  static constexpr int SCALES = 16 * RS;                        // offset of the 16 per-token scales (ROWS576)
  static constexpr int SLOT = 16 * RS + 64;                     // bytes of one ring slot
  static constexpr int DEPTH = 3;                               // ring slots per wave
};

// Dword 3 of a raw buffer resource on gfx9-family chips (no format conversion, no swizzle).
constexpr int kBufferFlags = 0x00020000;

// Two query dwords of a ROWS640 latent step: bytes 2i + bb of the step hold dim (bb ? y : x)[i], i < 4, from the
// bf16 pairs x = x0 | x1 << 16 and y = y0 | y1 << 16.
__device__ __forceinline__ void interleave_pairs(uint32_t x, uint32_t y, uint32_t& d0, uint32_t& d1) {
  d0 = (x & 0xffffu) | (y << 16);
  d1 = (x >> 16) | (y & 0xffff0000u);
}

// WIDE: a sparse pool past 4 GiB, whose rows take 64-bit addresses (every other pool is read through 32-bit buffer
// offsets).
template <int FMT, int WAVES, bool FINAL, bool WIDE>
__global__ __launch_bounds__(64 * WAVES) void mla_decode_kernel(MlaArgs a) {
  using Geo = TileGeo<FMT>;
  constexpr int NDMA = Geo::NDMA;
  constexpr int SLOT = Geo::SLOT;
  constexpr int RS = Geo::RS;
  constexpr int DEPTH = Geo::DEPTH;
  constexpr int ROWB = RowFmt<FMT>::kRowBytes;
  constexpr bool SPARSE = FMT == ROWS640;
  constexpr int NT = 64 * WAVES;
  static_assert(WAVES == 4, "the merge splits the 8 latent blocks over 4 waves");
  typedef __attribute__((address_space(3))) void lds_void;
  typedef __attribute__((address_space(3))) uint8_t lds_u8;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int g4 = lane >> 4;
  const int li = lane & 15;
  const int hg = blockIdx.y;  // 16-head group
  const int nh = min(16, a.H - 16 * hg);

  // LDS: each wave's ring of DEPTH tile slots (after the tile loop: the merge exchange), the sparse row ids, and the
  // waves' softmax statistics.
  __shared__ __attribute__((aligned(16))) uint8_t sm_ring[WAVES][DEPTH][SLOT];
  __shared__ int32_t sm_rowid[SPARSE ? kMlaMaxSplitKeys : 1];
  __shared__ float sm_m[WAVES][16];
  __shared__ float sm_l[WAVES][16];
  // The own row in the pool's row format (its bytes stand for all 16 keys of a tile with row stride 0), then its
  // scale repeated 16 times at kOwnScales.
  constexpr int kOwnScales = 640;
  __shared__ __attribute__((aligned(16))) uint8_t sm_own[kOwnScales + 64];
  __shared__ uint4 sm_q[18][64];
  // The merge exchange: block idx < 6 of sender w, 256 float4.
  static_assert(sizeof(float4) * WAVES * 6 * 256 <= sizeof(sm_ring), "the merge exchange lives in the ring");
  auto xchg = [&](int w, int idx) -> float4* { return reinterpret_cast<float4*>(&sm_ring[0][0][0]) + (w * 6 + idx) * 256; };

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
    if ((int32_t)blockIdx.x < a.work_n) {  // the plan's map, from the kernel arguments
    const uint32_t e = a.work[blockIdx.x];
    b = (int32_t)(e >> 6);
    split = (int32_t)(e & 63u);
  } else {
    locate_work<16>(a.seq_lens, a.B, 0, a.split_tiles, (int32_t)blockIdx.x, b, split);
  }
  }
  b = __builtin_amdgcn_readfirstlane(b);
  split = __builtin_amdgcn_readfirstlane(split);
  if (b < 0 || split >= max(a.max_splits, 1)) return;  // (past the plan's count: dropped, no write out of bounds)

  const int32_t khi = SPARSE ? a.n_indices : ld_const(a.seq_lens + b) - 1;
  const int32_t t_first = split * a.split_tiles;
  const int32_t t_last = min(t_first + a.split_tiles, (khi + 15) / 16);
  const int32_t kbase = t_first * 16;
  const int32_t* trow = a.table + (int64_t)b * a.table_stride;

  // ---- prologue: the split's block-table entries (paged), the query operand, the own row ----
  int32_t pg0 = -1, pg1 = -1, col0 = 0;
  if constexpr (!SPARSE) {
    // a split spans at most 128 table columns: at most 2048 keys, pages of at least 16
    col0 = kbase / a.P;
    const int32_t col_end = min((t_last * 16 - 1) / a.P + 1, a.table_width);
    if (col0 + lane < col_end) pg0 = trow[col0 + lane];
    if (col0 + 64 + lane < col_end) pg1 = trow[col0 + 64 + lane];
  }
  // The query operand of every QK step, in lane order: sm_q[s][lane] holds the 8 bf16 lane (g4, li) feeds in step s
  // (head li). ROWS576: step pair k is chunk 4 k + g4 = dims 16 (4 k + g4) .. + 15 (rope for k = 8). ROWS640: steps
  // 0, 1 are rope chunk 4 s + g4 (dims 8 (4 s + g4) .. + 7); step pair k > 0 is latent chunk m = 4 (k - 1) + g4,
  // whose byte 2 i + bb holds dim 256 a + 128 bb + p0 + i.
  // The paged format DMAs it in the tile loop's prologue, behind the first tiles' loads; the sparse format interleaves
  // pairs and fills it here.
  for (int e = tid; SPARSE && e < 18 * 64; e += NT) {
    const int s = e >> 6, ln = e & 63, eg4 = ln >> 4;
    const int32_t h = min(16 * hg + (ln & 15), a.H - 1);  // absent heads read a real head; their results are dropped
    const uint16_t* qlp = a.ql + ((int64_t)b * a.H + h) * kLatent;
    const uint16_t* qpp = a.qpe + ((int64_t)b * a.H + h) * kRope;
    uint4 w;
    if constexpr (FMT == ROWS576) {
      const int d = 16 * (4 * (s >> 1) + eg4) + 8 * (s & 1);
      w = d < kLatent ? ld16(qlp + d) : ld16(qpp + (d - kLatent));
    } else if (s < 2) {
      w = ld16(qpp + 8 * (4 * s + eg4));
    } else {
      const int m = 4 * ((s >> 1) - 1) + eg4;
      const int a0 = (16 * m) >> 8, p0 = ((16 * m) & 255) >> 1;
      const uint4 x = ld16(qlp + 256 * a0 + p0), y = ld16(qlp + 256 * a0 + 128 + p0);
      if (s & 1) {
        interleave_pairs(x.z, y.z, w.x, w.y);
        interleave_pairs(x.w, y.w, w.z, w.w);
      } else {
        interleave_pairs(x.x, y.x, w.x, w.y);
        interleave_pairs(x.y, y.y, w.z, w.w);
      }
    }
    sm_q[s][ln] = w;
  }
  // The own row is attended by one wave (the one with the fewest tiles) before its tiles, while their first loads are
  // in flight. Paged, that is a wave of the row's last split: the row's shortest, so the own row's quantization (a
  // few microseconds of one wave that its workgroup waits for) lands on a workgroup that finishes early. Sparse rows
  // split evenly, and split 0 takes it (measured faster there). Its bf16 elements 8 lane .. + 7 and
  // 8 (lane + 64) .. + 7 (lane < 8) and its pool slot load here, with the compiler's other prologue loads.
  const int32_t ntiles = t_last - t_first;
  const int32_t own_split = (!SPARSE && khi > 0) ? ((khi + 15) / 16 - 1) / a.split_tiles : 0;
  const bool own_wave = split == own_split && wave == ((ntiles % WAVES) == 0 ? WAVES - 1 : ntiles % WAVES);
  uint4 own0 = make_uint4(0, 0, 0, 0), own1 = make_uint4(0, 0, 0, 0);
  int64_t own_slot = -1;
  uint32_t own_q[4] = {0, 0, 0, 0};  // ROWS576: the quantized bytes of those elements, for the deferred pool store
  float own_s = 1.0f;
  if (own_wave) {
    const uint16_t* src = a.own + (int64_t)b * 576;
    own0 = ld16(src + 8 * lane);
    if (lane < 8) own1 = ld16(src + 8 * (lane + 64));
    if (!SPARSE && hg == 0 && a.new_slots) own_slot = redirect_slot(a.new_slots[b], a.num_blocks * a.P);
  }

  // Sparse: every index of the split to a row id (-1: skipped), all loads of a stage in flight together.
  if constexpr (SPARSE) {
    constexpr int KPT = kMlaMaxSplitKeys / NT;
    const int32_t nkeys = (t_last - t_first) * 16;
    const int32_t qpos = a.positions[b];
    const int64_t n_rows = a.num_blocks * a.P;
    int32_t pos[KPT];
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int32_t k = tid + i * NT, key = kbase + k;
      pos[i] = (k < nkeys && key < khi) ? a.indices[(int64_t)b * a.n_indices + key] : -1;
    }
    int32_t ent[KPT];
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      ent[i] = -1;
      if (pos[i] >= 0 && pos[i] <= qpos && pos[i] / a.P < a.table_width) ent[i] = trow[pos[i] / a.P];
    }
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int32_t k = tid + i * NT;
      if (k >= nkeys) continue;
      int32_t row = -1;
      if (ent[i] >= 0 && (int64_t)ent[i] < a.num_blocks) {
        const int64_t r = (int64_t)ent[i] * a.P + pos[i] % a.P;
        if (r < n_rows) row = (int32_t)r;
      }
      sm_rowid[k] = row;
    }
    __syncthreads();
  }

  // Each lane's source chunk for every DMA of a tile: LDS chunk o = 64 j + lane is chunk o % STRIDE of row
  // o / STRIDE (the pad chunk repeats the row's last chunk; rows past the tile only occur on switched-off lanes).
  // Offsets are 32-bit against a uniform base, so the DMAs take the scalar-base + vector-offset address form.
  uint32_t dma_src[NDMA];
#pragma unroll
  for (int j = 0; j < NDMA; ++j) {
    const uint32_t o = 64 * j + lane;
    const uint32_t r = min(o / Geo::STRIDE, 15u);
    const uint32_t c = min(o % Geo::STRIDE, (uint32_t)Geo::CHUNKS - 1);
    dma_src[j] = SPARSE ? (r << 16) | (16 * c) : r * ROWB + 16 * c;
  }

  // Paged: the first slot of tile `tile` and whether its page is real (uniform).
  auto tile_row0 = [&](int32_t tile, bool& ok) -> int64_t {
    const int32_t key0 = tile * 16;
    const int32_t col = key0 / a.P - col0;  // < 128
    const int32_t page = __builtin_amdgcn_readlane(col < 64 ? pg0 : pg1, col & 63);
    ok = page >= 0 && (int64_t)page < a.num_blocks;
    return ok ? (int64_t)page * a.P + key0 % a.P : 0;
  };
  // The valid keys of tile `tile` (bit k: key k), uniform.
  auto tile_mask = [&](int32_t tile) -> uint32_t {
    if constexpr (SPARSE) {
      return (uint32_t)(__ballot(sm_rowid[tile * 16 - kbase + li] >= 0) & 0xffffull);
    } else {
      bool ok;
      (void)tile_row0(tile, ok);
      const int32_t nvalid = ok ? min(16, khi - tile * 16) : 0;
      return nvalid >= 16 ? 0xffffu : (1u << nvalid) - 1u;
    }
  };
  // Issue the loads of tile `tile` into the ring slot at dst: NDMA DMAs, and the per-token scales (paged).
  // The DMAs read through buffer resources (a uniform base and size in SGPRs, a 32-bit offset per lane); the
  // sparse rows of a pool past 4 GiB take 64-bit addresses instead.
  const __amdgpu_buffer_rsrc_t pool_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)a.cache, (short)0, WIDE ? 0 : (int)(uint32_t)(a.num_blocks * a.P * ROWB), kBufferFlags);
  auto issue = [&](uint32_t d, int32_t tile) {  // d: the slot's LDS address
    if constexpr (SPARSE) {
      const int32_t k0 = tile * 16 - kbase;
#pragma unroll
      for (int j = 0; j < NDMA; ++j) {
        const int32_t row = max(sm_rowid[k0 + (int32_t)(dma_src[j] >> 16)], 0);
        if (j < NDMA - 1 || lane < Geo::TAIL) {
          if constexpr (!WIDE)
            dma_buffer16(pool_rsrc, d + 1024 * j, (uint32_t)row * ROWB + (dma_src[j] & 0xffffu));
          else
            dma_global16(a.cache + (int64_t)row * ROWB + (dma_src[j] & 0xffffu), d + 1024 * j);
        }
      }
    } else {
      bool ok;
      const int64_t row0 = tile_row0(tile, ok);
      const __amdgpu_buffer_rsrc_t rk =
          __builtin_amdgcn_make_buffer_rsrc((void*)(a.cache + row0 * ROWB), (short)0, 16 * ROWB, kBufferFlags);
#pragma unroll
      for (int j = 0; j < NDMA; ++j)
        if (j < NDMA - 1 || lane < Geo::TAIL)
          dma_buffer16(rk, d + 1024 * j, dma_src[j]);
      // the tile's 16 per-token scales (consecutive like its rows), in slot order
      const __amdgpu_buffer_rsrc_t rs =
          __builtin_amdgcn_make_buffer_rsrc((void*)(a.row_scale + row0), (short)0, 64, kBufferFlags);
      if (lane < 16)
        dma_buffer4(rs, d + Geo::SCALES, 4u * (uint32_t)key_of(lane));
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

  // A masked key's latent bytes may be anything, and a stale NaN or Inf would survive p = 0 in PV: a tile with masked
  // keys has their latent bytes zeroed in LDS first (its scores and scales are masked by selects).
  auto sanitize = [&](uint8_t* T, uint32_t vmask) {
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int idx = lane + 64 * it, r = idx >> 5, c = idx & 31;
      if (!((vmask >> r) & 1u))
        *reinterpret_cast<uint4*>(T + r * RS + (SPARSE ? 128 : 0) + 16 * c) = make_uint4(0, 0, 0, 0);
    }
  };
  // PV of one tile: O^T += V^T P^T over 32 d-tiles. Lane (g4, j) points the transposing read at slot
  // 4 g4 + (j / 2) % 4, bytes 16 (j / 8) + 8 (j % 2) of each 32-byte step, so that rows 0 .. 3 of its group's 8x16
  // byte matrix are slots 4 g4 .. 4 g4 + 3 at bytes 32 s .. 32 s + 15 and rows 4 .. 7 the same slots 16 bytes on.
  // (rs: the tile's LDS row stride; 0 for the own row standing for all 16 keys.)
  auto pv = [&](const uint8_t* T, const uint32_t (&pop)[2], int rs) {
    const uint8_t* Tv = T + key_of(4 * g4 + ((li >> 1) & 3)) * rs + (SPARSE ? 128 : 0) + 16 * (li >> 3) + 8 * (li & 1);
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const uint2 t = lds_read_tr8(Tv + 32 * s);
      uint32_t op[2];
      fp8x4_to_bf16x4(t.x, op[0], op[1]);
      acc[s >> 1][2 * (s & 1)] = mfma_16x16x16_bf16(op, pop, acc[s >> 1][2 * (s & 1)]);
      fp8x4_to_bf16x4(t.y, op[0], op[1]);
      acc[s >> 1][2 * (s & 1) + 1] = mfma_16x16x16_bf16(op, pop, acc[s >> 1][2 * (s & 1) + 1]);
    }
  };

  // Per-token scales of slots 4 g4 .. 4 g4 + 3 from the tile's 16 scales at S (1 for the sparse format).
  auto key_scales = [&](const uint8_t* S, float (&ks)[4]) {
    ks[0] = ks[1] = ks[2] = ks[3] = 1.0f;
    if constexpr (!SPARSE) {
      const float4 s4 = *reinterpret_cast<const float4*>(S + 16 * g4);
      ks[0] = s4.x, ks[1] = s4.y, ks[2] = s4.z, ks[3] = s4.w;
    }
  };
  // The tile's scores in the log2 domain (x[r]: slot 4 g4 + r, head li; -inf when masked) and their maximum per head.
  auto scores = [&](const uint8_t* T, uint32_t vmask, float (&x)[4], float& tmax, int rs, const uint8_t* S) {
    float ks[4];
    [[clang::always_inline]] key_scales(S, ks);
    // S^T = K Q^T: three accumulators keep three independent MFMA chains in flight
    const uint8_t* Tq = T + key_of(li) * rs + 16 * g4;
    f32x4_t scp[3] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int k = 0; k < 9; ++k) {
      f32x4_t& sc = scp[k % 3];
      if constexpr (SPARSE) {
        if (k == 0) {
          // steps 0 and 1: the bf16 rope, one chunk each
          const uint4 w0 = *reinterpret_cast<const uint4*>(Tq);
          const uint4 w1 = *reinterpret_cast<const uint4*>(Tq + 64);
          const uint32_t a0[4] = {w0.x, w0.y, w0.z, w0.w}, a1[4] = {w1.x, w1.y, w1.z, w1.w};
          const uint4 q0 = sm_q[0][lane], q1 = sm_q[1][lane];
          const uint32_t b0[4] = {q0.x, q0.y, q0.z, q0.w}, b1[4] = {q1.x, q1.y, q1.z, q1.w};
          sc = mfma_16x16x32_bf16(a0, b0, sc);
          sc = mfma_16x16x32_bf16(a1, b1, sc);
          continue;
        }
      }
      const uint4 w = *reinterpret_cast<const uint4*>(Tq + (SPARSE ? 128 + 64 * (k - 1) : 64 * k));
      uint32_t op0[4], op1[4];
      fp8x4_to_bf16x4(w.x, op0[0], op0[1]);
      fp8x4_to_bf16x4(w.y, op0[2], op0[3]);
      fp8x4_to_bf16x4(w.z, op1[0], op1[1]);
      fp8x4_to_bf16x4(w.w, op1[2], op1[3]);
      const uint4 q0 = sm_q[2 * k][lane], q1 = sm_q[2 * k + 1][lane];
      const uint32_t b0[4] = {q0.x, q0.y, q0.z, q0.w}, b1[4] = {q1.x, q1.y, q1.z, q1.w};
      sc = mfma_16x16x32_bf16(op0, b0, sc);
      sc = mfma_16x16x32_bf16(op1, b1, sc);
    }
    const f32x4_t sc = scp[0] + scp[1] + scp[2];
    tmax = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool ok = (vmask >> key_of(4 * g4 + r)) & 1u;
      x[r] = ok ? sc[r] * base_scale * ks[r] : -INFINITY;
      tmax = fmaxf(tmax, x[r]);
    }
    tmax = max_across_groups(tmax);
  };
  // Online softmax with a lazily moved reference maximum m_ref: a head moves it only when a tile's maximum passes it
  // by more than the slack (the probabilities stay below 2^slack), and then the accumulators are rescaled.
  auto needs_rescale = [&](float tmax) { return __any(tmax > m_ref + kMlaRescaleSlack); };
  auto rescale = [&](float tmax) {
    asm volatile("" ::: "memory");  // keeps the branch a branch: the compiler must not run the 128 multiplies always
    const float m_new = tmax > m_ref + kMlaRescaleSlack ? tmax : m_ref;
    const float alpha = __builtin_amdgcn_exp2f(m_ref - m_new);
    m_ref = m_new;
    l_run *= alpha;
#pragma unroll
    for (int q = 0; q < 8; ++q)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[q][r] *= alpha;
  };
  // The tile's probabilities against m_ref, folded into the row sum and, through PV, the accumulators.
  auto accumulate = [&](uint8_t* T, uint32_t vmask, const float (&x)[4], int rs, const uint8_t* S) {
    if (rs != 0 && vmask != 0xffffu) [[clang::always_inline]] sanitize(T, vmask);
    float ks[4];
    [[clang::always_inline]] key_scales(S, ks);
    float pw[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool ok = (vmask >> key_of(4 * g4 + r)) & 1u;
      const float p = __builtin_amdgcn_exp2f(x[r] - m_ref);
      l_run += p;
      // V is dequantized through P: p' = p * scale(key); a masked key has p = 0
      pw[r] = ok ? p * ks[r] : 0.0f;
    }
    const uint32_t pop[2] = {pack_bf16x2(pw[0], pw[1]), pack_bf16x2(pw[2], pw[3])};
    [[clang::always_inline]] pv(T, pop, rs);
  };

  // ---- the tile loop: wave w takes tiles t_first + w + WAVES i through its ring of DEPTH slots; DEPTH - 1 tiles'
  // loads are in flight while one computes ----
  {
    // VMEM operations one tile issues: its DMAs, plus the per-token scale DMA of the paged format
    constexpr int PER_TILE = NDMA + (SPARSE ? 0 : 1);
    static_assert((DEPTH - 1) * PER_TILE < 64, "vmcnt range");
    const int32_t t0 = t_first + wave;
    const int32_t mine = t0 < t_last ? (t_last - t0 + WAVES - 1) / WAVES : 0;
    const uint32_t ring = lds_address((lds_void*)(lds_u8*)&sm_ring[wave][0][0]);
    // The compiler's own loads (block table, query, indices) complete here, in a wait it sees (vmcnt(0): encoded
    // vmcnt 0, expcnt 7, lgkmcnt 15), before any DMA is in flight; otherwise it could wait for them again inside the
    // loop, and such a wait would drain the DMAs.
    __builtin_amdgcn_s_waitcnt(0x0f70);
    if constexpr (!SPARSE) {
      // the query operand, step s by wave s % WAVES: sm_q[s][lane] = dims 16 (4 (s / 2) + g4) + 8 (s % 2) .. + 7
      const int32_t h = min(16 * hg + li, a.H - 1);
      const uint16_t* qlp = a.ql + ((int64_t)b * a.H + h) * kLatent;
      const uint16_t* qpp = a.qpe + ((int64_t)b * a.H + h) * kRope;
      for (int s = wave; s < 18; s += WAVES) {
        const int d = 16 * (4 * (s >> 1) + g4) + 8 * (s & 1);
        dma_global16(d < kLatent ? qlp + d : qpp + (d - kLatent), lds_address((lds_void*)(lds_u8*)&sm_q[s][0]));
      }
    }
#pragma unroll
    for (int i = 0; i < DEPTH - 1; ++i)
      if (i < mine) issue(ring + i * SLOT, t0 + i * WAVES);
    // The own row, quantized as the store quantizes it, into sm_own in the pool's row format (LDS and registers only:
    // nothing here may add to the VMEM count the waits below rely on).
    if (own_wave) {
      const uint32_t w[8] = {own0.x, own0.y, own0.z, own0.w, own1.x, own1.y, own1.z, own1.w};
      if constexpr (FMT == ROWS576) {
        float m = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          m = fmaxf(m, fabsf(bf16_bits_to_f32(w[j] & 0xffffu)));
          m = fmaxf(m, fabsf(bf16_bits_to_f32(w[j] >> 16)));
        }
        own_s = scale_from_absmax(wave_max(m));
#pragma unroll
        for (int part = 0; part < 2; ++part) {
          if (part == 1 && lane >= 8) continue;
          uint32_t o[2] = {0, 0};
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const uint32_t bits = (w[part * 4 + (i >> 1)] >> ((i & 1) * 16)) & 0xffffu;
            o[i >> 2] |= quantize_e4m3fn(bits, own_s) << ((i & 3) * 8);
          }
          own_q[2 * part] = o[0];
          own_q[2 * part + 1] = o[1];
          *reinterpret_cast<uint2*>(&sm_own[8 * (lane + 64 * part)]) = make_uint2(o[0], o[1]);
        }
        if (lane < 16) reinterpret_cast<float*>(&sm_own[kOwnScales])[lane] = own_s;
      } else {
        // [rope 64 | latent 512] bf16 -> [bf16(rope / kv_scale) | e4m3fn(latent / kv_scale), permuted]
#pragma unroll
        for (int part = 0; part < 2; ++part) {
          if (part == 1 && lane >= 8) continue;
          const int ch = lane + 64 * part;  // 8-element chunk of the own row
          if (ch < 8) {
            uint32_t o[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const uint32_t lo = f32_to_bf16_bits(bf16_bits_to_f32(w[part * 4 + i] & 0xffffu) / a.kv_scale);
              const uint32_t hi = f32_to_bf16_bits(bf16_bits_to_f32(w[part * 4 + i] >> 16) / a.kv_scale);
              o[i] = lo | (hi << 16);
            }
            *reinterpret_cast<uint4*>(&sm_own[16 * ch]) = make_uint4(o[0], o[1], o[2], o[3]);
          } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              const uint32_t bits = (w[part * 4 + (i >> 1)] >> ((i & 1) * 16)) & 0xffffu;
              sm_own[128 + latent_byte_of_dim(8 * (ch - 8) + i)] = (uint8_t)quantize_e4m3fn(bits, a.kv_scale);
            }
          }
        }
      }
    }
    if constexpr (!SPARSE) {
      // every wave's query DMAs have landed (the tiles' may stay in flight), then the operand is complete
      static_assert(DEPTH == 3, "the waits below count two tiles");
      if (mine >= 2) wait_vmcnt<2 * PER_TILE>();
      else if (mine == 1) wait_vmcnt<PER_TILE>();
      else wait_vmcnt<0>();
      __syncthreads();
    }
    // The own row as key 0 of a one-key tile whose 16 rows all read sm_own (row stride 0; the other keys masked).
    if (own_wave) {
      float xo[4], to;
      [[clang::always_inline]] scores(&sm_own[0], 1u, xo, to, 0, &sm_own[kOwnScales]);
      if (needs_rescale(to)) [[clang::always_inline]] rescale(to);
      [[clang::always_inline]] accumulate(&sm_own[0], 1u, xo, 0, &sm_own[kOwnScales]);
    }
    // The rare rescale sits outside the inner loop, so inside it the accumulators are only ever MFMA operands and
    // keep their registers: a tile whose scores need a rescale leaves the loop before its PV and re-enters after it.
    int slot = 0;
    int32_t i = 0;
    bool pending = false;
    float x[4], tmax = -INFINITY;
    uint32_t vm = 0;
    while (true) {
      for (; i < mine; ++i) {
        uint8_t* T = &sm_ring[wave][slot][0];
        if (!pending) {
          // issue tile i + DEPTH - 1 into the slot tile i - 1 freed, then wait until tile i's loads have landed:
          // the loads of the tiles after it may stay in flight
          const int32_t ahead = mine - 1 - i;
          if (ahead >= DEPTH - 1) {
            issue(ring + (slot == 0 ? DEPTH - 1 : slot - 1) * SLOT, t0 + (i + DEPTH - 1) * WAVES);
            wait_vmcnt<(DEPTH - 1) * PER_TILE>();
          } else if (DEPTH > 3 && ahead == 2) {
            wait_vmcnt<2 * PER_TILE>();
          } else if (ahead == 1) {
            wait_vmcnt<PER_TILE>();
          } else {
            wait_vmcnt<0>();
          }
          vm = tile_mask(t0 + i * WAVES);
          [[clang::always_inline]] scores(T, vm, x, tmax, RS, T + Geo::SCALES);
          if (needs_rescale(tmax)) {
            pending = true;
            break;
          }
        }
        pending = false;
        [[clang::always_inline]] accumulate(T, vm, x, RS, T + Geo::SCALES);
        slot = slot == DEPTH - 1 ? 0 : slot + 1;
      }
      if (!pending) break;
      [[clang::always_inline]] rescale(tmax);
    }
    wait_vmcnt<0>();
  }

  // ---- the own row's pool store (ROWS576), deferred to here so that no store sits among the DMAs in flight ----
  if (own_wave && own_slot >= 0) {
#pragma unroll
    for (int part = 0; part < 2; ++part) {
      if (part == 1 && lane >= 8) continue;
      *reinterpret_cast<uint2*>(a.cache + own_slot * 576 + 8 * (lane + 64 * part)) =
          make_uint2(own_q[2 * part], own_q[2 * part + 1]);
    }
    if (lane == 0) a.row_scale[own_slot] = own_s;
  }

  // ---- merge: a common maximum per head; wave w sums latent blocks 2 w, 2 w + 1 over the waves and writes them ----
  const float l_w = sum_across_groups(l_run);
  if (g4 == 0) {
    sm_m[wave][li] = m_ref;
    sm_l[wave][li] = l_w;
  }
  __syncthreads();  // every wave is past its tile loop: the ring's space is free for the exchange
  float M = sm_m[0][li];
#pragma unroll
  for (int w = 1; w < WAVES; ++w) M = fmaxf(M, sm_m[w][li]);
  float L = 0.0f;
#pragma unroll
  for (int w = 0; w < WAVES; ++w) L += __builtin_amdgcn_exp2f(sm_m[w][li] - M) * sm_l[w][li];
  const float f = __builtin_amdgcn_exp2f(m_ref - M);
  // exchange slot of (sender w, block q not its own): [w][q < 2 w ? q : q - 2][r][lane]
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    if (q / 2 == wave) continue;
    const int idx = q < 2 * wave ? q : q - 2;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const f32x4_t v = acc[q][r] * f;
      xchg(wave, idx)[r * 64 + lane] = make_float4(v[0], v[1], v[2], v[3]);
    }
  }
  __syncthreads();
  const int32_t h = 16 * hg + li;
  const int32_t S = a.max_splits;
  const float oscale = SPARSE ? a.kv_scale : 1.0f;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    if (q / 2 != wave) continue;
    f32x4_t v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      v[r] = acc[q][r] * f;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) {
        if (w == wave) continue;
        const int idx = q < 2 * w ? q : q - 2;
        const float4 t = xchg(w, idx)[r * 64 + lane];
        v[r][0] += t.x;
        v[r][1] += t.y;
        v[r][2] += t.z;
        v[r][3] += t.w;
      }
    }
    if (li >= nh) continue;
    // v[r][r']: latent byte beta + r' with beta = 64 q + 16 r + 4 g4; ROWS640 bytes beta, beta + 2 are dims d0, d0 + 1
    // and bytes beta + 1, beta + 3 dims d0 + 128, d0 + 129
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] *= oscale;
    if constexpr (FINAL) {
      const float inv = 1.0f / L;
      uint16_t* dst = a.out + ((int64_t)b * a.H + h) * kLatent;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int beta = 64 * q + 16 * r + 4 * g4;
        if constexpr (!SPARSE) {
          *reinterpret_cast<uint2*>(dst + beta) =
              make_uint2(pack_bf16x2(v[r][0] * inv, v[r][1] * inv), pack_bf16x2(v[r][2] * inv, v[r][3] * inv));
        } else {
          const int d0 = latent_dim_of_byte(beta);
          *reinterpret_cast<uint32_t*>(dst + d0) = pack_bf16x2(v[r][0] * inv, v[r][2] * inv);
          *reinterpret_cast<uint32_t*>(dst + d0 + 128) = pack_bf16x2(v[r][1] * inv, v[r][3] * inv);
        }
      }
      if (a.lse_out && q == 0 && g4 == 0) a.lse_out[(int64_t)b * a.H + h] = (M + __log2f(L)) * 0.6931471805599453f;
    } else {
      const int64_t row = ((int64_t)b * S + split) * a.H + h;
      float* dst = a.ws_o + row * kLatent;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int beta = 64 * q + 16 * r + 4 * g4;
        if constexpr (!SPARSE) {
          *reinterpret_cast<float4*>(dst + beta) = make_float4(v[r][0], v[r][1], v[r][2], v[r][3]);
        } else {
          const int d0 = latent_dim_of_byte(beta);
          *reinterpret_cast<float2*>(dst + d0) = make_float2(v[r][0], v[r][2]);
          *reinterpret_cast<float2*>(dst + d0 + 128) = make_float2(v[r][1], v[r][3]);
        }
      }
      if (q == 0 && g4 == 0) *reinterpret_cast<float2*>(a.ws_ml + row * 2) = make_float2(M, L);
    }
  }
}

// Merge of a row's splits, two waves per (row, head): out = sum_s e_s o_s / sum_s e_s l_s, lse = M + log(sum), with
// e_s = exp2(m_s - M). Lane s holds split s's weight; wave w, lane i the latent dims 256 w + 4 i .. + 3. The
// partials stream in chunks of 16 splits, each chunk's loads all in flight together (the first before the weights
// are known).
template <int FMT>
__global__ __launch_bounds__(128) void mla_combine_kernel(MlaArgs a) {
  constexpr bool SPARSE = FMT == ROWS640;
  constexpr int CH = 16;
  const int b = blockIdx.x, h = blockIdx.y, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int32_t S = a.max_splits;
  // The first chunk of partials and every split's (m, l) load before the row's split count is known: they are
  // bounded by the workspace's S splits per row, not by the count, so they do not wait for the seq_lens load. Entries
  // past the count are dropped by selects.
  const int64_t row0 = (int64_t)b * S * a.H + h;
  const float* ob = a.ws_o + row0 * kLatent + 256 * w + 4 * lane;
  const int64_t sstride = (int64_t)a.H * kLatent;
  float4 x[CH];
#pragma unroll
  for (int k = 0; k < CH; ++k)
    if (k < S) x[k] = *reinterpret_cast<const float4*>(ob + k * sstride);
  float2 ml = make_float2(-INFINITY, 0.0f);
  if (lane < S) ml = *reinterpret_cast<const float2*>(a.ws_ml + (row0 + (int64_t)lane * a.H) * 2);
  const int32_t n = min(SPARSE ? splits_of<16>(a.n_indices + 1, 0, a.split_tiles)
                               : splits_of<16>(ld_const(a.seq_lens + b), 0, a.split_tiles),
                        S);
  if (n == 0) return;  // a row with no prior key: the lone-row kernel writes it
  const float m = lane < n ? ml.x : -INFINITY, l = lane < n ? ml.y : 0.0f;
  const float M = wave_max(m);
  const float e = lane < n ? __builtin_amdgcn_exp2f(m - M) : 0.0f;
  const float den = wave_sum(e * l);
  float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int32_t base = 0; base < n; base += CH) {
    if (base > 0) {
#pragma unroll
      for (int k = 0; k < CH; ++k)
        if (base + k < n) x[k] = *reinterpret_cast<const float4*>(ob + (base + k) * sstride);
    }
#pragma unroll
    for (int k = 0; k < CH; ++k) {
      if (base + k < n) {
        const float es = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), base + k));
        o.x += es * x[k].x, o.y += es * x[k].y, o.z += es * x[k].z, o.w += es * x[k].w;
      }
    }
  }
  const float inv = 1.0f / den;
  *reinterpret_cast<uint2*>(a.out + ((int64_t)b * a.H + h) * kLatent + 256 * w + 4 * lane) =
      make_uint2(pack_bf16x2(o.x * inv, o.y * inv), pack_bf16x2(o.z * inv, o.w * inv));
  if (a.lse_out && w == 0 && lane == 0) a.lse_out[(int64_t)b * a.H + h] = (M + __log2f(den)) * 0.6931471805599453f;
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
  hipEvent_t t0, t1;
  if (grid_x > 0) {
    timing_events(0, &t0, &t1);
    const dim3 grid(grid_x, groups);
    // only a sparse pool can take the 64-bit kernel (W is false for the paged format)
    constexpr bool W = FMT == ROWS640;
    const bool wide = W && a.num_blocks * a.P * (int64_t)RowFmt<FMT>::kRowBytes > 0xffffffffll;
    if (a.max_splits <= 1) {
      if (wide) hipExtLaunchKernelGGL((mla_decode_kernel<FMT, 4, true, W>), grid, dim3(256), 0, s, t0, t1, 0, a);
      else hipExtLaunchKernelGGL((mla_decode_kernel<FMT, 4, true, false>), grid, dim3(256), 0, s, t0, t1, 0, a);
    } else {
      if (wide) hipExtLaunchKernelGGL((mla_decode_kernel<FMT, 4, false, W>), grid, dim3(256), 0, s, t0, t1, 0, a);
      else hipExtLaunchKernelGGL((mla_decode_kernel<FMT, 4, false, false>), grid, dim3(256), 0, s, t0, t1, 0, a);
    }
  }
  if (a.max_splits > 1) {
    timing_events(1, &t0, &t1);
    hipExtLaunchKernelGGL((mla_combine_kernel<FMT>), dim3(a.B, a.H), dim3(128), 0, s, t0, t1, 0, a);
  }
  if (any_lone) hipLaunchKernelGGL((mla_lone_row_kernel<FMT>), dim3(a.B, groups), dim3(256), 0, s, a);
  timing_end_call();
}

static int check_plan(const sna_split_plan* plan, int32_t B, const char* what) {
  if (!plan || plan->tile != 16 || plan->split_tiles < 1 || plan->n_work < 0 || plan->max_splits < 0 ||
      plan->batch != B)
    return fail(SNA_ERR_INVALID_ARGUMENT, "%s: missing or foreign split plan (made for %d rows)", what,
                plan ? plan->batch : -1);
  if (plan->split_tiles * 16 > kMlaMaxSplitKeys)
    return fail(SNA_ERR_INVALID_ARGUMENT, "%s: a split of %d keys exceeds the kernel's %d", what,
                plan->split_tiles * 16, kMlaMaxSplitKeys);
  return check_work_map(plan, B, what);
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
  a.work_n = plan->work_n;
  for (int32_t i = 0; i < plan->work_n; ++i) a.work[i] = plan->work[i];
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
  a.work_n = plan->work_n;
  for (int32_t i = 0; i < plan->work_n; ++i) a.work[i] = plan->work[i];
  a.ws_o = need > 0 ? ws : nullptr;
  a.ws_ml = need > 0 ? ws + (int64_t)B * plan->max_splits * num_heads * kLatent : nullptr;
  a.out = (uint16_t*)ctx_out;
  a.lse_out = lse_out;
  launch_mla<ROWS640>(a, groups, per * B, per == 0, (hipStream_t)stream);
  return check_launch("mla_decode_sparse");
}
