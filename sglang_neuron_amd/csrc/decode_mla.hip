// Absorbed-MLA decode (paged, per-token FP8 scale) and DSA sparse decode (index lists over 640-byte packed rows):
// online softmax with all 16 heads of a head group in one wave, MFMA for QK^T and PV, in one launch per decode.
//
// Row formats:
//   ROWS576  [latent 512 | k_pe 64] e4m3fn, one fp32 dequantization scale per token slot (row_scale).
//   ROWS1152 [latent 512 | k_pe 64] bf16, no scale (the reference's DeepSeek-V2 pool).
//   ROWS640  [k_pe 64 bf16 | latent 512 e4m3fn, permuted], one per-tensor kv_scale. Latent dim c = 256a + 128b + p
//            sits at latent byte 256a + 2p + b.
//
// Work: a stream split. Every row's key tiles (16 keys; at least one per row) are laid end to end and workgroup w
// (4 waves, one per CU) takes tiles [cta_start[w], cta_start[w + 1]) of that sequence, equal counts for every
// workgroup, so the workgroups end together. Its range is one or more segments, each inside one row; per segment the
// 4 waves take the tiles round-robin through their rings of LDS slots, filled by global->LDS DMA, so the in-flight
// bytes cost no registers. Paged: a tile is 16 consecutive slots of one page (the page size is a multiple of 16), one
// contiguous 9 KB run; the segment's block-table entries sit in four VGPRs and a tile's page is a readlane. Sparse:
// the segment's indices are resolved to row ids in LDS first (index -> block -> row). The segment holding a row's last
// tile attends the row's own row: one wave quantizes it as the store does and attends it as a one-key tile.
//
// A segment that is a whole row writes the row's output. A row split over S workgroups is merged in the same launch:
// each of its workgroups writes its partial (unnormalized context, max and sum per head) through to memory and counts
// itself in the row's arrival word. The row's eight 64-dim latent blocks are shared out by arrival order: a workgroup
// that sees the row complete (the last to arrive, or one still polling the word when it completes) merges its blocks
// over the S partials in one pass; an owner whose bounded polls run out retracts its blocks in the same word, and the
// last to arrive merges those. The last workgroup of the launch to finish returns every word to zero.
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
#include <algorithm>
#include <type_traits>

#include "sna_device.h"
#include "sna_host.h"

namespace sna {

enum { ROWS576 = 0, ROWS640 = 1, ROWS1152 = 2 };

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
  const int32_t* indices;    // sparse [B, n_indices]
  int32_t n_indices;
  int32_t spec;              // sparse: query tokens per sequence (rows s * spec .. + spec - 1 share table row s)
  const int32_t* positions;  // sparse [B]
  const uint16_t* own;       // [B, 576] bf16: ROWS576 [latent | rope], ROWS640 [rope | latent]
  const int64_t* new_slots;  // store the own rows there (NULL: the caller has stored them)
  int32_t B, H, P, groups;
  int64_t num_blocks;
  float sm_scale;
  int32_t n_ctas;      // workgroups per head group
  int32_t wait_polls;  // polls of a row's arrival counter by a workgroup that published a partial
  float* ws_o;         // [2 n_ctas, H, 512] partial contexts (unnormalized; ROWS640 in latent-byte order)
  float* ws_ml;        // [2 n_ctas, H, 2] their (max, sum), log2 domain
  int32_t* ws_cnt;     // arrival words [kStreamMaxCounters], (unused) [kStreamMaxCounters], finished workgroups,
                       // status (each a 64-byte line)
  const int32_t* seq_lens;  // paged [B] (device): a device-split launch cuts its stream from them
  uint16_t* out;
  float* lse_out;
  uint32_t cta_start[SNA_MAX_CTAS + 1];  // the stream split (sna_split_plan)
  uint32_t cta_row_off[SNA_MAX_CTAS];    // row << 16 | tile offset in it (32-bit words take scalar loads)
  int32_t row_keys[SNA_MAX_PLAN_ROWS];   // keys per row: paged seq_len - 1, sparse n_indices
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
  static constexpr int kLatentBytes = 512;
};
template <>
struct RowFmt<ROWS640> {
  static constexpr int kRowBytes = 640;
  static constexpr int kLatentBytes = 512;
};
template <>
struct RowFmt<ROWS1152> {
  static constexpr int kRowBytes = 1152;
  static constexpr int kLatentBytes = 1024;
};

// Tile geometry in LDS. A tile is 16 key rows; chunk c (16 bytes) of row r sits at LDS chunk r * STRIDE + c, with
// STRIDE = CHUNKS + 1: the pad chunk puts rows 1 apart 20 (ROWS576) or 36 (ROWS640, ROWS1152) banks apart and rows 4
// apart 16 banks apart, so the QK reads (16 rows, one 16-byte chunk each) and the PV reads (4 rows x 64 bytes per lane group)
// are free of bank conflicts, and every LDS address is a per-lane base plus a constant. NDMA wave-wide DMAs fill a
// slot: lane i of DMA j fills LDS chunk 64 j + i. A pad chunk loads a duplicate of its row's last chunk; the lanes of
// the last DMA past the tile are switched off. ROWS576 tiles bring their 16 per-token scales along in one more DMA.
template <int FMT>
struct TileGeo {
  static constexpr int CHUNKS = RowFmt<FMT>::kRowBytes / 16;
  static constexpr int STRIDE = CHUNKS + 1;
  static constexpr int RS = 16 * STRIDE;                        // LDS row stride, bytes
  static constexpr int NDMA = (16 * STRIDE + 63) / 64;          // 10 or 11
  static constexpr int TAIL = 16 * STRIDE - 64 * (NDMA - 1);    // active lanes of the last DMA
  static constexpr int SCALES = 16 * RS;                        // offset of the 16 per-token scales (ROWS576)
  static constexpr int SLOT = 16 * RS + 64;                     // bytes of one ring slot
  // ring slots per wave: two (FP8 rows with staged tiles measured 42.3 µs on the cfg3 batch against 43.3 with three
  // and 44.7 with four, and the sparse gathers of the cfg5 batch 20.0 against 21.1 with three: fewer loads
  // outstanding per wave stream faster)
  static constexpr int DEPTH = 2;
};
// Slots the ring array holds per wave: its depth, or three 16-key FP8 slots' bytes, which the waves' merge exchange
// (96 KB) reuses after the tile loop.
template <int FMT>
constexpr int kRingSlots = FMT == ROWS1152 ? TileGeo<FMT>::DEPTH : 3;

// Dword 3 of a raw buffer resource on gfx9-family chips (no format conversion, no swizzle).
constexpr int kBufferFlags = 0x00020000;
// The cache-policy operand of a raw buffer access for device scope on gfx950: SC1 (bit 4), the bit device-scope
// atomic loads and stores carry.
constexpr int kCachePolicyDevice = 0x10;

// Two query dwords of a ROWS640 latent step: bytes 2i + bb of the step hold dim (bb ? y : x)[i], i < 4, from the
// bf16 pairs x = x0 | x1 << 16 and y = y0 | y1 << 16.
__device__ __forceinline__ void interleave_pairs(uint32_t x, uint32_t y, uint32_t& d0, uint32_t& d1) {
  d0 = (x & 0xffffu) | (y << 16);
  d1 = (x >> 16) | (y & 0xffff0000u);
}

// One 640-byte DSA row packed from its bf16 [rope 64 | latent 512] source into LDS at dst, by the 64 lanes of a wave,
// bit for bit as kv_store_dsa_kernel packs it: lane l quantizes latent bytes 8 l .. 8 l + 7, lanes 0 .. 15 the rope.
__device__ __forceinline__ void pack_row640(const uint16_t* src, uint8_t* dst, float kv_scale, int lane) {
  uint32_t o[2] = {0, 0};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int32_t beta = 8 * lane + i, a0 = beta >> 8, rem = beta & 255;
    o[i >> 2] |= quantize_e4m3fn(src[64 + (a0 << 8) + ((rem & 1) << 7) + (rem >> 1)], kv_scale) << ((i & 3) * 8);
  }
  *reinterpret_cast<uint2*>(dst + 128 + 8 * lane) = make_uint2(o[0], o[1]);
  if (lane < 16) {
    const uint2 w = ld8(src + 4 * lane);
    const uint32_t r0 = f32_to_bf16_bits(bf16_bits_to_f32(w.x & 0xffffu) / kv_scale) |
                        (f32_to_bf16_bits(bf16_bits_to_f32(w.x >> 16) / kv_scale) << 16);
    const uint32_t r1 = f32_to_bf16_bits(bf16_bits_to_f32(w.y & 0xffffu) / kv_scale) |
                        (f32_to_bf16_bits(bf16_bits_to_f32(w.y >> 16) / kv_scale) << 16);
    *reinterpret_cast<uint2*>(dst + 8 * lane) = make_uint2(r0, r1);
  }
}

// The rows' new slots in a 512-entry open-addressing table in LDS (key: pool row, value: the highest batch row that
// stores there, the one whose bytes a gather of that slot sees, since the rows are stored in order): B <= 256 keys, so
// every probe sequence meets an empty entry.
constexpr int kSlotHash = 512;
__device__ __forceinline__ uint32_t slot_hash(int32_t row) { return ((uint32_t)row * 2654435761u) >> 23; }
__device__ __forceinline__ int32_t slot_lookup(const int32_t* keys, const int32_t* vals, int32_t row) {
  for (uint32_t h = slot_hash(row);; h = (h + 1) & (kSlotHash - 1)) {
    const int32_t k = keys[h];
    if (k == row) return vals[h];
    if (k == -1) return -1;
  }
}

// Partials cross workgroups (and so the chip's per-XCD L2s) inside one launch: they are written and read with device
// scope (sc1: coherent across the XCDs), through buffer resources over the workspace.
__device__ __forceinline__ void store_dev16(__amdgpu_buffer_rsrc_t r, uint32_t off, float4 v) {
  typedef float f32x4v __attribute__((ext_vector_type(4)));
  __builtin_amdgcn_raw_buffer_store_b128(f32x4v{v.x, v.y, v.z, v.w}, r, off, 0, kCachePolicyDevice);
}
__device__ __forceinline__ void store_dev8(__amdgpu_buffer_rsrc_t r, uint32_t off, float2 v) {
  typedef float f32x2v __attribute__((ext_vector_type(2)));
  __builtin_amdgcn_raw_buffer_store_b64(f32x2v{v.x, v.y}, r, off, 0, kCachePolicyDevice);
}
__device__ __forceinline__ float4 load_dev16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCachePolicyDevice);
  return make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3]));
}
__device__ __forceinline__ float2 load_dev8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kCachePolicyDevice);
  return make_float2(__uint_as_float(v[0]), __uint_as_float(v[1]));
}

// The numbers of workgroups (of n) whose range starts at or before global tiles x0 and x1: the stream split's
// starts, one per lane in four independent loads (so one memory round trip; a device split's from LDS, where the
// entries past its ranges hold the stream's end), counted by ballots.
template <bool DEV>
__device__ __forceinline__ void ctas_starting_by(const MlaArgs& a, const uint32_t* dev_starts, uint32_t x0, uint32_t x1,
                                                 int32_t& n0, int32_t& n1) {
  static_assert(SNA_MAX_CTAS <= 256, "four loads of 64 starts");
  const int lane = threadIdx.x & 63;
  uint32_t c[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int k = 64 * i + lane;
    if constexpr (DEV) c[i] = dev_starts[k];
    else c[i] = k < a.n_ctas ? a.cta_start[k] : 0xffffffffu;
  }
  int32_t s0 = 0, s1 = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s0 += __popcll(__ballot(c[i] <= x0));
    s1 += __popcll(__ballot(c[i] <= x1));
  }
  n0 = __builtin_amdgcn_readfirstlane(s0);
  n1 = __builtin_amdgcn_readfirstlane(s1);
}

// ---- the stream split cut on the device (a plan from a bound), so that one captured launch serves any lengths ----

// Inclusive prefix sums over the wave's 64 lanes of four values per lane, scanned together (shuffles up).
__device__ __forceinline__ void wave_incl_scan4(uint32_t (&v)[4]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    uint32_t t[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) t[i] = (uint32_t)__shfl_up((int)v[i], d, 64);
    if (lane >= d) {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] += t[i];
    }
  }
}

// Wave 0 of every workgroup of a device-split launch cuts the same stream split from the device's seq_lens (the
// arithmetic is deterministic, so every workgroup gets the same one): the rows' key counts (seq_len - 1, held to the
// table's width and the stream's 65535 tiles per row) into keys[b]; the ranges' starts into cs[w] (cs[w] = the
// stream's end for w at or past the split's n, and cs[256] too); row << 16 | tile offset into cro[w]; n into *n_out.
// With a workgroup for every row (B <= n, n = min(launched workgroups, tiles)) rows are apportioned whole: the least
// piece length T with sum_b ceil(tiles_b / T) <= n is found by bisection, and row b is cut into ceil(tiles_b / T)
// equal pieces (the same longest piece as the host planner's greedy apportionment, within a tile); otherwise the
// stream is cut into n equal ranges. tmp: 5 x 256 words of LDS scratch.
__device__ void device_split(const MlaArgs& a, uint32_t* cs, uint32_t* cro, int32_t* keys, int32_t* n_out,
                             uint32_t* tmp) {
  const int lane = threadIdx.x & 63;
  const int32_t B = a.B;
  const int32_t kmax = (int32_t)min((int64_t)a.table_width * a.P, (int64_t)65535 * 16);
  uint32_t tiles[4], first[4], mx = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int32_t r = lane + 64 * i;
    tiles[i] = 0;
    if (r < B) {
      const int32_t k = min(max(a.seq_lens[r] - 1, 0), kmax);
      keys[r] = k;
      tiles[i] = (uint32_t)max((k + 15) >> 4, 1);
    }
    first[i] = tiles[i];
    mx = max(mx, tiles[i]);
  }
  wave_incl_scan4(first);
  uint32_t total = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t part = (uint32_t)__shfl((int)first[i], 63, 64);
    first[i] = total + first[i] - tiles[i];
    total += part;
  }
  const uint32_t n = min((uint32_t)gridDim.x, total);
  uint32_t* t_first = tmp;
  uint32_t* t_tiles = tmp + 256;
  uint32_t* t_pieces = tmp + 512;
  uint32_t* t_pfirst = tmp + 768;
  uint32_t* mark = tmp + 1024;  // row + 1 at the first workgroup of a row (0 elsewhere)
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int32_t r = lane + 64 * i;
    mark[r] = 0;
    if (r < B) {
      t_first[r] = first[i];
      t_tiles[r] = tiles[i];
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  const bool whole = (uint32_t)B <= n;
  uint32_t n_split = n;
  if (whole) {
    mx = (uint32_t)wave_max((float)mx);
    uint32_t lo = max(1u, (total + n - 1) / n), hi = mx;
    if (n > (uint32_t)B) hi = min(hi, (total + (n - B) - 1) / (n - B));  // feasible: sum <= total / T + B <= n
    lo = min(lo, hi);
    while (lo < hi) {
      const uint32_t mid = (lo + hi) >> 1;
      const float rt = 1.0f / (float)mid;
      uint32_t sum = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) sum += ceil_div_small(tiles[i], mid, rt);
      if ((uint32_t)wave_sum((float)sum) <= n) hi = mid;
      else lo = mid + 1;
    }
    const float rt = 1.0f / (float)lo;
    uint32_t pieces[4], pf[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) pf[i] = pieces[i] = ceil_div_small(tiles[i], lo, rt);
    wave_incl_scan4(pf);
    n_split = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t part = (uint32_t)__shfl((int)pf[i], 63, 64);
      pf[i] = n_split + pf[i] - pieces[i];
      n_split += part;
      const int32_t r = lane + 64 * i;
      if (r < B) {
        t_pieces[r] = pieces[i];
        t_pfirst[r] = pf[i];
        mark[pf[i]] = (uint32_t)r + 1;  // every row has a piece, so the firsts are distinct
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int32_t r = lane + 64 * i;
      // the first range starting at or after the row's first tile: ceil(first * n / total)
      const uint32_t w0 = r < B ? (uint32_t)(((uint64_t)first[i] * n + total - 1) / total) : n;
      if (w0 < n) atomicMax(&mark[w0], (uint32_t)r + 1);
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  // a workgroup's row: the prefix maximum of the marks (lane l holds workgroups 4 l .. 4 l + 3)
  uint32_t m[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) m[j] = mark[4 * lane + j];
#pragma unroll
  for (int j = 1; j < 4; ++j) m[j] = max(m[j], m[j - 1]);
  uint32_t run = m[3];
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t t = (uint32_t)__shfl_up((int)run, d, 64);
    if (lane >= d) run = max(run, t);
  }
  uint32_t before = (uint32_t)__shfl_up((int)run, 1, 64);
  if (lane == 0) before = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t w = 4 * lane + j;
    if (w < n_split) {
      const uint32_t r = max(m[j], before) - 1;
      const uint32_t off = whole ? (w - t_pfirst[r]) * t_tiles[r] / t_pieces[r]
                                 : (uint32_t)((uint64_t)w * total / n) - t_first[r];
      cs[w] = t_first[r] + off;
      cro[w] = r << 16 | off;
    } else {
      cs[w] = total;
      cro[w] = 0;
    }
  }
  if (lane == 0) {
    cs[256] = total;
    *n_out = (int32_t)n_split;
  }
}

// Merge of up to NC latent blocks (chunks[i]: dims 64 c .. 64 c + 63; -1 = none) of row b, head group hg, over its S
// partials: those of workgroups w0 .. w0 + S - 1 (workgroup w0's is its second slot when its range starts before the
// row). Thread (j, q) = (tid / 16, tid % 16) takes head 16 hg + j, dims 64 c + 4 q .. + 3 of each block. First the
// row's max M and sum L: lane q of a head's 16 lanes loads the (max, sum) of partials q, q + 16, ... (four rounds of
// loads in flight at once, the first NK partials' contexts with them) and keeps them in `lds` ([16][256] float2, its
// own entries), where each max is then replaced by the partial's weight 2^(m_k - M). Then the contexts are added in
// partial order with those final weights, NK partials' loads in flight at a time. No running rescale: the sums are
// the same bits whatever NC and NK, so a block's result does not depend on which workgroup merges it.
template <bool SPARSE, int NC, int NK>
__device__ void merge_chunks(const MlaArgs& a, __amdgpu_buffer_rsrc_t ro, __amdgpu_buffer_rsrc_t rml, int32_t b, int hg,
                             int32_t w0, bool w0_second, int32_t S, const int (&chunks)[NC], float2* lds) {
  static_assert(NC * NK <= 64, "a group's loads stay in registers");
  static_assert(SNA_MAX_CTAS <= 16 * 16, "16 rounds of 16 partials cover a row");
  const int tid = threadIdx.x, j = tid >> 4, q = tid & 15;
  const int32_t h = min(16 * hg + j, a.H - 1);  // absent heads merge a real head's data; their results are dropped
  auto slot_of = [&](int32_t k) -> int32_t { return 2 * (w0 + k) + ((k == 0 && w0_second) ? 1 : 0); };
  auto ml_of = [&](int32_t k) -> float2 {
    return k < S ? load_dev8(rml, (uint32_t)(((int64_t)slot_of(k) * a.H + h) * 8)) : make_float2(kNegBig, 0.0f);
  };
  float4 x[NC][NK];
  auto load_group = [&](int32_t base) {
#pragma unroll
    for (int k = 0; k < NK; ++k) {
      if (base + k >= S) continue;
      const int64_t prow = ((int64_t)slot_of(base + k) * a.H + h) * kLatent + 4 * q;
#pragma unroll
      for (int i = 0; i < NC; ++i)
        if (chunks[i] >= 0) x[i][k] = load_dev16(ro, (uint32_t)((prow + 64 * chunks[i]) * 4));
    }
  };
  load_group(0);
  const int32_t R = (S + 15) >> 4;
  float m = kNegBig;
  for (int32_t r0 = 0; r0 < R; r0 += 4) {
    float2 ml[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ml[i] = ml_of(16 * (r0 + i) + q);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (r0 + i >= R) break;
      lds[(r0 + i) * 256 + tid] = ml[i];
      m = fmaxf(m, ml[i].x);
    }
  }
  const float M = row16_max(m);
  float l = 0.0f;
  for (int32_t r = 0; r < R; ++r) {
    const float2 ml = lds[r * 256 + tid];
    const float e = __builtin_amdgcn_exp2f(ml.x - M);
    l += e * ml.y;
    lds[r * 256 + tid].x = e;
  }
  const float L = row16_sum(l);
  __syncthreads();  // every lane's weights are in LDS
  float4 o[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) o[i] = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int32_t base = 0; base < S; base += NK) {
    if (base > 0) load_group(base);
#pragma unroll
    for (int k = 0; k < NK; ++k) {
      const int32_t kk = base + k;
      if (kk >= S) continue;
      const float ek = lds[(kk >> 4) * 256 + 16 * j + (kk & 15)].x;
#pragma unroll
      for (int i = 0; i < NC; ++i)
        if (chunks[i] >= 0) o[i].x += ek * x[i][k].x, o[i].y += ek * x[i][k].y, o[i].z += ek * x[i][k].z,
                            o[i].w += ek * x[i][k].w;
    }
  }
  if (16 * hg + j >= a.H) return;  // (the caller's next barrier ends the weights' use of the LDS)
  const float inv = 1.0f / L;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    if (chunks[i] < 0) continue;
    uint16_t* dst = a.out + ((int64_t)b * a.H + h) * kLatent;
    const int beta = 64 * chunks[i] + 4 * q;  // the partials' latent byte of o[i].x
    if constexpr (!SPARSE) {
      *reinterpret_cast<uint2*>(dst + beta) =
          make_uint2(pack_bf16x2(o[i].x * inv, o[i].y * inv), pack_bf16x2(o[i].z * inv, o[i].w * inv));
    } else {
      // bytes beta .. beta + 3 of a ROWS640 latent are dims d0, d0 + 128, d0 + 1, d0 + 129
      const int d0 = latent_dim_of_byte(beta);
      *reinterpret_cast<uint32_t*>(dst + d0) = pack_bf16x2(o[i].x * inv, o[i].z * inv);
      *reinterpret_cast<uint32_t*>(dst + d0 + 128) = pack_bf16x2(o[i].y * inv, o[i].w * inv);
    }
    if (SPARSE && a.lse_out && chunks[i] == 0 && q == 0)
      a.lse_out[(int64_t)b * a.H + h] = (M + __log2f(L)) * 0.6931471805599453f;
  }
}

// The blocks of `mask` (bit c: latent block c) merged over the row's S partials: one block with 16 partials' loads in
// flight, several with 8. lds: 32 KB of LDS for the merge's weights.
template <bool SPARSE>
__device__ void merge_mask(const MlaArgs& a, __amdgpu_buffer_rsrc_t ro, __amdgpu_buffer_rsrc_t rml, int32_t b, int hg,
                           int32_t w0, bool w0_second, int32_t S, uint32_t mask, float2* lds) {
  if (__popc(mask) == 1) {
    const int chunks[1] = {__builtin_ctz(mask)};
    merge_chunks<SPARSE, 1, 16>(a, ro, rml, b, hg, w0, w0_second, S, chunks, lds);
    return;
  }
  int chunks[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) chunks[i] = (mask >> i) & 1u ? i : -1;
  merge_chunks<SPARSE, 8, 8>(a, ro, rml, b, hg, w0, w0_second, S, chunks, lds);
}

// WIDE: a sparse pool past 4 GiB, whose rows take 64-bit addresses (every other pool is read through 32-bit buffer
// offsets). MULTI: some workgroup's range spans several rows (a plan with more rows than workgroups); without it each
// range is one segment, and the kernel is the segment loop's body once (the loop's carried state costs the one-segment
// kernel its scalar registers). DEV: the stream split is cut from the device's seq_lens at the start of the launch
// (device_split), not taken from the plan; the grid is the plan's bound, and workgroups past the split's ranges only
// count themselves finished. XORD: the XCD-aware order of the pieces (below; the sparse kernel with spec > 1).
template <int FMT, bool WIDE, bool MULTI, bool DEV = false, bool XORD = false>
__global__ __launch_bounds__(256) void mla_decode_kernel(MlaArgs a) {
  constexpr int WAVES = 4;
  using Geo = TileGeo<FMT>;
  constexpr int NDMA = Geo::NDMA;
  constexpr int SLOT = Geo::SLOT;
  constexpr int RS = Geo::RS;
  constexpr int DEPTH = Geo::DEPTH;
  constexpr int ROWB = RowFmt<FMT>::kRowBytes;
  constexpr bool SPARSE = FMT == ROWS640;
  constexpr bool BF16 = FMT == ROWS1152;
  constexpr int NT = 64 * WAVES;
  typedef __attribute__((address_space(3))) void lds_void;
  typedef __attribute__((address_space(3))) uint8_t lds_u8;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int g4 = lane >> 4;
  const int li = lane & 15;
  const int hg = blockIdx.y;  // 16-head group
  const int nh = min(16, a.H - 16 * hg);
  // With spec query tokens per sequence (MTP verify), sibling tokens read mostly the same rows (the recent window,
  // overlapping index lists, each other's own rows): the XCD-aware order puts a sequence's consecutive pieces on one
  // XCD, so those rows come from its L2 (cfg5 at spec 8: 53.6 -> 50.3-51.1 us). With one token per row it measured
  // neutral (MLA) or slightly slower (DSA), so those keep the launch order, in their own instantiations.
  const int32_t w = XORD ? (int32_t)xcd_order(blockIdx.x, gridDim.x) : (int32_t)blockIdx.x;

  // LDS: each wave's ring of DEPTH tile slots (after a segment's tile loop: the merge exchange), the sparse row ids,
  // the waves' softmax statistics, the own row, the query operand (bf16 rows: in registers, the ring takes the
  // space), and a broadcast word.
  __shared__ __attribute__((aligned(16))) uint8_t sm_ring[WAVES][kRingSlots<FMT>][SLOT];
  __shared__ int32_t sm_rowid[SPARSE ? kMlaMaxSplitKeys : 1];
  __shared__ uint4 sm_q[SPARSE ? 18 : 1][64];
  // FP8 rows: the head group's query as it lies in memory, DMA'd once per workgroup ([16][512] latent, then [16][64]
  // rope, bf16)
  __shared__ __attribute__((aligned(16))) uint8_t sm_qraw[FMT == ROWS576 ? 18432 : 16];
  __shared__ float sm_m[WAVES][16];
  __shared__ float sm_l[WAVES][16];
  // The own row in the pool's row format (its bytes stand for all 16 keys of a tile with row stride 0), then its
  // scale repeated 16 times at kOwnScales (ROWS576).
  constexpr int kOwnScales = BF16 ? 1152 : 640;
  __shared__ __attribute__((aligned(16))) uint8_t sm_own[kOwnScales + 64];
  __shared__ int32_t sm_word;
  // The merge exchange: block idx < 6 of sender w, 256 float4.
  static_assert(sizeof(float4) * WAVES * 6 * 256 <= sizeof(sm_ring), "the merge exchange lives in the ring");
  auto xchg = [&](int sw, int idx) -> float4* {
    return reinterpret_cast<float4*>(&sm_ring[0][0][0]) + (sw * 6 + idx) * 256;
  };

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
  const __amdgpu_buffer_rsrc_t pool_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)a.cache, (short)0, WIDE ? 0 : (int)(uint32_t)(a.num_blocks * a.P * ROWB), kBufferFlags);
  const float base_scale = a.sm_scale * kLog2e * (SPARSE ? a.kv_scale : 1.0f);

  // ---- a device split: cut by wave 0 into LDS (the ring is scratch until the first DMA) ----
  __shared__ uint32_t sm_cs[DEV ? SNA_MAX_CTAS + 1 : 1];
  __shared__ uint32_t sm_cro[DEV ? SNA_MAX_CTAS : 1];
  __shared__ int32_t sm_keys[DEV ? SNA_MAX_PLAN_ROWS : 1];
  __shared__ int32_t sm_nsplit;
  if constexpr (DEV) {
    static_assert(sizeof(sm_ring) >= 5 * 256 * 4, "the split's scratch fits the ring");
    if (wave == 0)
      device_split(a, sm_cs, sm_cro, sm_keys, &sm_nsplit, reinterpret_cast<uint32_t*>(&sm_ring[0][0][0]));
    __syncthreads();
  }
  auto cta_start = [&](int32_t k) -> uint32_t {
    if constexpr (DEV) return __builtin_amdgcn_readfirstlane(sm_cs[k]);
    else return a.cta_start[k];
  };
  auto row_keys = [&](int32_t r) -> int32_t {
    if constexpr (DEV) return __builtin_amdgcn_readfirstlane(sm_keys[r]);
    else return a.row_keys[r];
  };
  const uint32_t cro_w = DEV ? __builtin_amdgcn_readfirstlane(sm_cro[w]) : a.cta_row_off[w];

  // ---- the workgroup's range of the stream, one segment (a piece of one row) at a time ----
  const uint32_t g_lo = cta_start(w), g_hi = cta_start(w + 1);
  int32_t b = (int32_t)(cro_w >> 16);
  uint32_t row_t0 = g_lo - (cro_w & 0xffffu);  // the global index of row b's first tile
  for (uint32_t g = g_lo; g < g_hi; ++b) {
    const int32_t khi = row_keys(b);  // the row's keys: positions [0, khi) (paged) or index entries (sparse)
    const uint32_t row_t1 = row_t0 + (uint32_t)max((khi + 15) >> 4, 1);
    const uint32_t s_hi = min(g_hi, row_t1);
    const int32_t t_first = (int32_t)(g - row_t0);
    const int32_t t_last = (int32_t)(s_hi - row_t0);
    const bool whole = g == row_t0 && s_hi == row_t1;   // the segment is the whole row: it writes the output
    const bool has_own = g == row_t0;                    // it holds the row's first tile: it attends the own row
    const bool first_seg = g == g_lo;                    // the partial slot: 2 w for the first segment, 2 w + 1 after
    // the row's first and last workgroups (for the merge of a split row), found with the prologue's loads
    int32_t wa, wb;
    ctas_starting_by<DEV>(a, sm_cs, row_t0, row_t1 - 1, wa, wb);
    --wa;
    --wb;
    const int32_t kbase = t_first * 16;
    // the row's sequence: its table row (sparse: spec query tokens per sequence)
    const int32_t seq = SPARSE ? b / a.spec : b;
    const int32_t* trow = a.table + (int64_t)seq * a.table_stride;
    const int32_t ntiles = t_last - t_first;

    // ---- prologue: the segment's block-table entries (paged), the query operand, the own row ----
    int32_t pg[4] = {-1, -1, -1, -1};
    int32_t col0 = 0;
    if constexpr (!SPARSE) {
      // the first 256 table columns of the segment in four VGPRs (bounded by the table only, so these loads do not
      // wait for the row's key count); a tile past them reads its entry itself
      col0 = kbase / a.P;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (col0 + 64 * r + lane < a.table_width) pg[r] = trow[col0 + 64 * r + lane];
    }
    // The query operand of every QK step, the 8 bf16 lane (g4, li) feeds in step s (head li). Paged formats: in
    // registers, qreg[s] = dims 16 (4 k + g4) + 8 (s % 2) .. + 7 for step pair k = s / 2 (rope for k = 8). ROWS640: in
    // LDS, sm_q[s][lane]: steps 0, 1 are rope chunk 4 s + g4 (dims 8 (4 s + g4) .. + 7); step pair k > 0 is latent
    // chunk m = 4 (k - 1) + g4, whose byte 2 i + bb holds dim 256 a + 128 bb + p0 + i (pairs interleaved here; the
    // workgroup's threads share the loads, which sit on a sparse row's critical path).
    // (The loads are issued here, with the other prologue loads; the LDS stores follow the index loads below, so
    // the query, the own row, the indices and the new slots share one round trip.)
    constexpr int QIT = SPARSE ? (18 * 64 + NT - 1) / NT : 1;
    uint4 qx[QIT], qy[QIT];
    if constexpr (SPARSE) {
#pragma unroll
      for (int it = 0; it < QIT; ++it) {
        const int e = tid + it * NT;
        const int s = e >> 6, ln = e & 63, eg4 = ln >> 4;
        const int32_t h = min(16 * hg + (ln & 15), a.H - 1);  // absent heads read a real head; their results are dropped
        const uint16_t* qlp = a.ql + ((int64_t)b * a.H + h) * kLatent;
        const uint16_t* qpp = a.qpe + ((int64_t)b * a.H + h) * kRope;
        qx[it] = qy[it] = make_uint4(0, 0, 0, 0);
        if (e < 18 * 64) {
          if (s < 2) {
            qx[it] = ld16(qpp + 8 * (4 * s + eg4));
          } else {
            const int m = 4 * ((s >> 1) - 1) + eg4;
            const int a0 = (16 * m) >> 8, p0 = ((16 * m) & 255) >> 1;
            qx[it] = ld16(qlp + 256 * a0 + p0);
            qy[it] = ld16(qlp + 256 * a0 + 128 + p0);
          }
        }
      }
    }
    // FP8 rows (FP8QK): QK runs on v_mfma_scale_f32_16x16x128_f8f6f4 for the latent dims, K's bytes straight from the
    // tile. Lane (g4, li) then supplies dims 128 kb + 32 g4 .. + 31 of latent block kb (kb < 4) of head li: its bf16
    // query values (loaded here as qreg[4 kb .. 4 kb + 3]) scaled by a power of two sc (the head's absolute maximum
    // into [128, 256)) and split exactly into two e4m3fn parts, hi + lo / 16, whose per-lane E8M0 B scales undo sc
    // (and lo's 1/16), so K . Q is the bf16 dot product accumulated in fp32. The rope dims stay bf16 (qreg[16],
    // qreg[17]: dims 16 g4 .. + 7 and 16 g4 + 8 .. + 15 of the rope) for two v_mfma_f32_16x16x32_bf16 steps.
    constexpr bool FP8QK = FMT == ROWS576;
    uint4 qreg[SPARSE ? 1 : 18];
    if constexpr (!SPARSE && !FP8QK) {
      const int32_t h = min(16 * hg + li, a.H - 1);
      const uint16_t* qlp = a.ql + ((int64_t)b * a.H + h) * kLatent;
      const uint16_t* qpp = a.qpe + ((int64_t)b * a.H + h) * kRope;
#pragma unroll
      for (int st = 0; st < 18; ++st) {
        const int d = FP8QK ? (st < 16 ? 128 * (st >> 2) + 32 * g4 + 8 * (st & 3) : kLatent + 16 * g4 + 8 * (st & 1))
                            : 16 * (4 * (st >> 1) + g4) + 8 * (st & 1);
        qreg[st] = ld16(d < kLatent ? qlp + d : qpp + (d - kLatent));
      }
    }
    uint32_t qhi[FP8QK ? 4 : 1][8], qlo[FP8QK ? 4 : 1][8];
    int32_t qs_hi = 127, qs_lo = 127;
    // the split of the latent query (after the first tiles' loads are issued, so that it runs under their latency)
    auto split_query = [&]() {
      if constexpr (FP8QK) {
        float amax = 0.0f;
#pragma unroll
        for (int st = 0; st < 16; ++st) {
          const uint32_t ww[4] = {qreg[st].x, qreg[st].y, qreg[st].z, qreg[st].w};
#pragma unroll
          for (int e = 0; e < 4; ++e)
            amax = fmaxf(amax, fmaxf(fabsf(bf16_bits_to_f32(ww[e] & 0xffffu)), fabsf(bf16_bits_to_f32(ww[e] >> 16))));
        }
        amax = max_across_groups(amax);
        // sc = 2^(7 - floor(log2 amax)): amax * sc in [128, 256); E8M0 scale of hi = 127 - log2 sc, of lo 4 less (the
        // exponent is held to [-116, 127], where sc and both E8M0 scales are representable; a head that small only
        // loses bits far below the tolerance)
        const int32_t ex = amax > 0.0f ? max((int32_t)((__float_as_uint(amax) >> 23) & 0xff) - 127, -116) : -7;
        const float sc = __uint_as_float((uint32_t)(127 + 7 - ex) << 23);
        qs_hi = 127 + ex - 7;
        qs_lo = qs_hi - 4;
#pragma unroll
        for (int st = 0; st < 16; ++st) {
          const uint32_t ww[4] = {qreg[st].x, qreg[st].y, qreg[st].z, qreg[st].w};
#pragma unroll
          for (int e2 = 0; e2 < 2; ++e2) {
            float h4[4], l4[4];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
              split_q(bf16_bits_to_f32(ww[2 * e2 + e] & 0xffffu) * sc, h4[2 * e], l4[2 * e]);
              split_q(bf16_bits_to_f32(ww[2 * e2 + e] >> 16) * sc, h4[2 * e + 1], l4[2 * e + 1]);
            }
            qhi[st >> 2][2 * (st & 3) + e2] = pack_e4m3fn_x4(h4[0], h4[1], h4[2], h4[3]);
            qlo[st >> 2][2 * (st & 3) + e2] = pack_e4m3fn_x4(l4[0], l4[1], l4[2], l4[3]);
          }
        }
      }
    };
    // the query operand of QK step st (8 bf16 of head li, as lane (g4, li) feeds them)
    auto q_op = [&](int st) -> uint4 {
      if constexpr (SPARSE) return sm_q[st][lane];
      else return qreg[st];
    };
    // The own row is attended by one wave (the one with the fewest tiles of the segment) before its tiles, while their
    // first loads are in flight. Its bf16 elements 8 lane .. + 7 and 8 (lane + 64) .. + 7 (lane < 8) and its pool slot
    // load here, with the compiler's other prologue loads.
    const bool own_wave = has_own && wave == ((ntiles % WAVES) == 0 ? WAVES - 1 : ntiles % WAVES);
    uint4 own0 = make_uint4(0, 0, 0, 0), own1 = make_uint4(0, 0, 0, 0);
    int64_t own_slot = -1;
    uint32_t own_q[4] = {0, 0, 0, 0};  // ROWS576: the quantized bytes of those elements, for the deferred pool store
    float own_s = 1.0f;
    if (own_wave) {
      const uint16_t* src = a.own + (int64_t)b * 576;
      own0 = ld16(src + 8 * lane);
      own1 = ld16(src + 8 * (min(lane, 7) + 64));  // lanes 8 .. 63 repeat lane 7's load (their own1 is unused)
      if (hg == 0 && a.new_slots) {
        // paged: an out-of-range slot goes to the reserved row 0, as kv_store_mla does; sparse: it is skipped, as
        // kv_store_dsa does
        const int64_t s0 = a.new_slots[b];
        own_slot = SPARSE ? ((s0 >= 0 && s0 < a.num_blocks * a.P) ? s0 : -1) : redirect_slot(s0, a.num_blocks * a.P);
      }
    }

    // Sparse: every index of the segment to a row id (-1: skipped), all loads of a stage in flight together. With
    // new_slots, a row that some batch row's own row is stored to in this launch becomes -2 - (that batch row): its
    // bytes are packed from the source row after the tile lands, so no gather depends on when the store lands.
    // With spec query tokens per sequence, a row's keys are its index list and then its spec - 1 siblings' own rows
    // (the other tokens of its sequence, in order), each -2 - (the sibling's batch row) at the sibling's position and
    // kept iff that position <= the row's: the reference appends every sibling's packed row
    // (mla_decode_attention_torch.py:89-103, 185-190) whatever its slot or table entry.
    if constexpr (SPARSE) {
      constexpr int KPT = kMlaMaxSplitKeys / NT;
      const int32_t nkeys = ntiles * 16;
      const int32_t qpos = a.positions[b];
      const int64_t n_rows = a.num_blocks * a.P;
      const int32_t jj = b - seq * a.spec;  // the row's token within its sequence
      int32_t pos[KPT], sib[KPT];
#pragma unroll
      for (int i = 0; i < KPT; ++i) {
        const int32_t k = tid + i * NT, key = kbase + k;
        pos[i] = -1;
        sib[i] = -1;
        if (k < nkeys && key < khi) {
          if (key < a.n_indices) {
            pos[i] = a.indices[(int64_t)b * a.n_indices + key];
          } else {
            const int32_t e = key - a.n_indices;
            sib[i] = seq * a.spec + e + (e >= jj ? 1 : 0);
            pos[i] = a.positions[sib[i]];
          }
        }
      }
      // thread e's row's new slot (B <= SNA_MAX_PLAN_ROWS = NT), loaded beside the indices: the barriers below wait
      // for every load in flight, so a load issued after one costs a round trip of its own
      static_assert(SNA_MAX_PLAN_ROWS <= NT, "one new slot per thread");
      const int64_t my_slot = (a.new_slots && tid < a.B) ? a.new_slots[tid] : -1;
      // the query operand's LDS stores (its loads were issued with the prologue's first loads)
#pragma unroll
      for (int it = 0; it < QIT; ++it) {
        const int e = tid + it * NT;
        if (e >= 18 * 64) continue;
        const int s = e >> 6, ln = e & 63;
        const uint4 x = qx[it], y = qy[it];
        uint4 wq = x;
        if (s >= 2) {
          if (s & 1) {
            interleave_pairs(x.z, y.z, wq.x, wq.y);
            interleave_pairs(x.w, y.w, wq.z, wq.w);
          } else {
            interleave_pairs(x.x, y.x, wq.x, wq.y);
            interleave_pairs(x.y, y.y, wq.z, wq.w);
          }
        }
        sm_q[s][ln] = wq;
      }
      // the new-slot table lives in the ring (unused until the tile loop)
      int32_t* hkey = reinterpret_cast<int32_t*>(&sm_ring[0][0][0]);
      int32_t* hval = hkey + kSlotHash;
      if (a.new_slots) {
        for (int e = tid; e < kSlotHash; e += NT) hkey[e] = hval[e] = -1;
        __syncthreads();
        if (my_slot >= 0 && my_slot < n_rows) {
          for (uint32_t h = slot_hash((int32_t)my_slot);; h = (h + 1) & (kSlotHash - 1)) {
            const int32_t prev = atomicCAS(&hkey[h], -1, (int32_t)my_slot);
            if (prev == -1 || prev == (int32_t)my_slot) {
              atomicMax(&hval[h], tid);
              break;
            }
          }
        }
        __syncthreads();
        // several rows storing to one slot: the last of them stores (the rows are stored in order)
        if (own_slot >= 0 && slot_lookup(hkey, hval, (int32_t)own_slot) != b) own_slot = -1;
      }
      int32_t ent[KPT];
#pragma unroll
      for (int i = 0; i < KPT; ++i) {
        ent[i] = -1;
        if (sib[i] < 0 && pos[i] >= 0 && pos[i] <= qpos && pos[i] / a.P < a.table_width) ent[i] = trow[pos[i] / a.P];
      }
#pragma unroll
      for (int i = 0; i < KPT; ++i) {
        const int32_t k = tid + i * NT;
        if (k >= nkeys) continue;
        int32_t row = -1;
        if (sib[i] >= 0) {
          if (pos[i] <= qpos) row = -2 - sib[i];  // a sibling's own row, packed from its source
        } else {
          if (ent[i] >= 0 && (int64_t)ent[i] < a.num_blocks) {
            const int64_t r = (int64_t)ent[i] * a.P + pos[i] % a.P;
            if (r < n_rows) row = (int32_t)r;
          }
          if (row >= 0 && a.new_slots) {
            const int32_t src = slot_lookup(hkey, hval, row);
            if (src >= 0) row = -2 - src;
          }
        }
        sm_rowid[k] = row;
      }
      __syncthreads();
    }

    // Paged: the first slot of tile `tile` and whether its page is real (uniform). The table entry is a readlane of
    // the prefetched columns, or a scalar load past them.
    auto tile_row0 = [&](int32_t tile, bool& ok) -> int64_t {
      const int32_t key0 = tile * 16;
      const int32_t col = key0 / a.P - col0;
      int32_t page;
      if (col < 256) {
        const int32_t v = col < 64 ? pg[0] : (col < 128 ? pg[1] : (col < 192 ? pg[2] : pg[3]));
        page = __builtin_amdgcn_readlane(v, col & 63);
      } else {
        page = col0 + col < a.table_width ? ld_const(trow + col0 + col) : -1;
      }
      ok = page >= 0 && (int64_t)page < a.num_blocks;
      return ok ? (int64_t)page * a.P + key0 % a.P : 0;
    };
    // The valid keys of tile `tile` (bit k: key k), uniform.
    auto tile_mask = [&](int32_t tile) -> uint32_t {
      if constexpr (SPARSE) {
        return (uint32_t)(__ballot(sm_rowid[tile * 16 - kbase + li] != -1) & 0xffffull);
      } else {
        bool ok;
        (void)tile_row0(tile, ok);
        const int32_t nvalid = ok ? max(min(16, khi - tile * 16), 0) : 0;
        return nvalid >= 16 ? 0xffffu : (1u << nvalid) - 1u;
      }
    };
    // Sparse: the keys of tile `tile` whose rows an own row is stored to in this launch (bit k: key k), uniform; their
    // LDS rows are packed from the source rows once the tile has landed.
    auto tile_aliases = [&](int32_t tile) -> uint32_t {
      if constexpr (SPARSE) return (uint32_t)(__ballot(sm_rowid[tile * 16 - kbase + li] <= -2) & 0xffffull);
      return 0u;
    };
    auto patch_aliases = [&](uint8_t* T, int32_t tile, uint32_t al) {
      for (; al; al &= al - 1) {
        const int r = __builtin_ctz(al);
        const int32_t src = -2 - sm_rowid[tile * 16 - kbase + r];
        pack_row640(a.own + (int64_t)src * 576, T + r * RS, a.kv_scale, lane);
      }
    };
    // Issue the loads of tile `tile` into the ring slot at dst: NDMA DMAs, and the per-token scales (paged).
    // The DMAs read through buffer resources (a uniform base and size in SGPRs, a 32-bit offset per lane); the
    // sparse rows of a pool past 4 GiB take 64-bit addresses instead.
    auto issue = [&](uint32_t d, int32_t tile) {  // d: the slot's LDS address
      if constexpr (SPARSE) {
        const int32_t k0 = tile * 16 - kbase;
        // every DMA's row id first, then the DMAs: a read between two DMAs (whose asm may touch memory) would wait
        // for its own round trip before the next DMA could issue
        int32_t row[NDMA];
#pragma unroll
        for (int j = 0; j < NDMA; ++j) row[j] = max(sm_rowid[k0 + (int32_t)(dma_src[j] >> 16)], 0);
#pragma unroll
        for (int j = 0; j < NDMA; ++j) {
          if (j < NDMA - 1 || lane < Geo::TAIL) {
            if constexpr (!WIDE)
              dma_buffer16(pool_rsrc, d + 1024 * j, (uint32_t)row[j] * ROWB + (dma_src[j] & 0xffffu));
            else
              dma_global16(a.cache + (int64_t)row[j] * ROWB + (dma_src[j] & 0xffffu), d + 1024 * j);
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
        if constexpr (FMT == ROWS576) {
          // the tile's 16 per-token scales (consecutive like its rows), in slot order
          const __amdgpu_buffer_rsrc_t rs =
              __builtin_amdgcn_make_buffer_rsrc((void*)(a.row_scale + row0), (short)0, 64, kBufferFlags);
          if (lane < 16)
            dma_buffer4(rs, d + Geo::SCALES, 4u * (uint32_t)key_of(lane));
        }
      }
    };

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
      constexpr int LCH = RowFmt<FMT>::kLatentBytes / 16;  // 16-byte latent chunks per row (32 or 64)
#pragma unroll
      for (int it = 0; it < LCH / 4; ++it) {
        const int idx = lane + 64 * it, r = idx / LCH, c = idx % LCH;
        if (!((vmask >> r) & 1u))
          *reinterpret_cast<uint4*>(T + r * RS + (SPARSE ? 128 : 0) + 16 * c) = make_uint4(0, 0, 0, 0);
      }
    };
    // PV of one tile: O^T += V^T P^T over 32 d-tiles. Lane (g4, j) points the transposing read at slot
    // 4 g4 + (j / 2) % 4, bytes 16 (j / 8) + 8 (j % 2) of each 32-byte step, so that rows 0 .. 3 of its group's 8x16
    // byte matrix are slots 4 g4 .. 4 g4 + 3 at bytes 32 s .. 32 s + 15 and rows 4 .. 7 the same slots 16 bytes on.
    // (rs: the tile's LDS row stride; 0 for the own row standing for all 16 keys.)
    auto pv = [&](const uint8_t* T, const uint32_t (&pop)[2], int rs) {
      if constexpr (BF16) {
        // bf16: lane (g4, j) points the transposing read at slot 4 g4 + j / 4, dims d0 + 4 (j % 4) .. + 3, so that row
        // k of its group's 4x16 matrix is slot 4 g4 + k at dims d0 .. d0 + 15 and lane (g4, i) receives dim d0 + i of
        // slots 4 g4 .. 4 g4 + 3: the A operand of d-tile d0 = 64 q + 16 r
        const uint8_t* Tb = T + key_of(4 * g4 + (li >> 2)) * rs + 8 * (li & 3);
#pragma unroll
        for (int q = 0; q < 8; ++q)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const uint2 t = lds_read_tr16(Tb + 2 * (64 * q + 16 * r));
            const uint32_t op[2] = {t.x, t.y};
            acc[q][r] = mfma_16x16x16_bf16(op, pop, acc[q][r]);
          }
        return;
      }
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
      if constexpr (FMT == ROWS576) {
        const float4 s4 = *reinterpret_cast<const float4*>(S + 16 * g4);
        ks[0] = s4.x, ks[1] = s4.y, ks[2] = s4.z, ks[3] = s4.w;
      }
    };
    // The tile's scores in the log2 domain (x[r]: slot 4 g4 + r, head li; -inf when masked) and their maximum per head.
    // FP8 rows: S^T of a tile from its 9 chunks of key key_of(li)'s row, kc[2 kb + j] = latent chunk 8 kb + 2 g4 + j
    // and kc[8] = rope chunk 32 + g4, in three independent MFMA chains
    auto qk_fp8 = [&](const uint4 (&kc)[9]) -> f32x4_t {
      f32x4_t sp[3] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const uint32_t a8[8] = {kc[2 * kb].x, kc[2 * kb].y, kc[2 * kb].z, kc[2 * kb].w,
                                kc[2 * kb + 1].x, kc[2 * kb + 1].y, kc[2 * kb + 1].z, kc[2 * kb + 1].w};
        f32x4_t& sc = sp[kb >> 1];
        sc = mfma_16x16x128_fp8(a8, qhi[kb], sc, qs_hi);
        sc = mfma_16x16x128_fp8(a8, qlo[kb], sc, qs_lo);
      }
      uint32_t op0[4], op1[4];
      fp8x4_to_bf16x4(kc[8].x, op0[0], op0[1]);
      fp8x4_to_bf16x4(kc[8].y, op0[2], op0[3]);
      fp8x4_to_bf16x4(kc[8].z, op1[0], op1[1]);
      fp8x4_to_bf16x4(kc[8].w, op1[2], op1[3]);
      const uint32_t b0[4] = {qreg[16].x, qreg[16].y, qreg[16].z, qreg[16].w};
      const uint32_t b1[4] = {qreg[17].x, qreg[17].y, qreg[17].z, qreg[17].w};
      sp[2] = mfma_16x16x32_bf16(op0, b0, sp[2]);
      sp[2] = mfma_16x16x32_bf16(op1, b1, sp[2]);
      return sp[0] + sp[1] + sp[2];
    };
    // the 9 chunks of a tile in LDS at T (row stride rs)
    auto load_chunks = [&](const uint8_t* T, int rs, uint4 (&kc)[9]) {
      const uint8_t* Tq = T + key_of(li) * rs;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int j = 0; j < 2; ++j) kc[2 * kb + j] = *reinterpret_cast<const uint4*>(Tq + 16 * (8 * kb + 2 * g4 + j));
      kc[8] = *reinterpret_cast<const uint4*>(Tq + 16 * (32 + g4));
    };
    auto scores = [&](const uint8_t* T, uint32_t vmask, float (&x)[4], float& tmax, int rs, const uint8_t* S) {
      float ks[4];
      [[clang::always_inline]] key_scales(S, ks);
      if constexpr (FP8QK) {
        uint4 kc[9];
        [[clang::always_inline]] load_chunks(T, rs, kc);
        const f32x4_t sc = qk_fp8(kc);
        tmax = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const bool ok = (vmask >> key_of(4 * g4 + r)) & 1u;
          x[r] = ok ? sc[r] * base_scale * ks[r] : -INFINITY;
          tmax = fmaxf(tmax, x[r]);
        }
        tmax = max_across_groups(tmax);
        return;
      }
      // S^T = K Q^T: three accumulators keep three independent MFMA chains in flight
      const uint8_t* Tq = T + key_of(li) * rs + 16 * g4;
      f32x4_t scp[3] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int k = 0; k < 9; ++k) {
        f32x4_t& sc = scp[k % 3];
        if constexpr (BF16) {
          // step pair k: dims 16 (4 k + g4) .. + 15 of key key_of(li), bytes 32 (4 k + g4) .. + 31 of its row
          const uint8_t* Tk = T + key_of(li) * rs + 32 * (4 * k + g4);
          const uint4 w0 = *reinterpret_cast<const uint4*>(Tk), w1 = *reinterpret_cast<const uint4*>(Tk + 16);
          const uint32_t a0[4] = {w0.x, w0.y, w0.z, w0.w}, a1[4] = {w1.x, w1.y, w1.z, w1.w};
          const uint4 q0 = q_op(2 * k), q1 = q_op(2 * k + 1);
          const uint32_t b0[4] = {q0.x, q0.y, q0.z, q0.w}, b1[4] = {q1.x, q1.y, q1.z, q1.w};
          sc = mfma_16x16x32_bf16(a0, b0, sc);
          sc = mfma_16x16x32_bf16(a1, b1, sc);
          continue;
        }
        if constexpr (SPARSE) {
          if (k == 0) {
            // steps 0 and 1: the bf16 rope, one chunk each
            const uint4 w0 = *reinterpret_cast<const uint4*>(Tq);
            const uint4 w1 = *reinterpret_cast<const uint4*>(Tq + 64);
            const uint32_t a0[4] = {w0.x, w0.y, w0.z, w0.w}, a1[4] = {w1.x, w1.y, w1.z, w1.w};
            const uint4 q0 = q_op(0), q1 = q_op(1);
            const uint32_t b0[4] = {q0.x, q0.y, q0.z, q0.w}, b1[4] = {q1.x, q1.y, q1.z, q1.w};
            sc = mfma_16x16x32_bf16(a0, b0, sc);
            sc = mfma_16x16x32_bf16(a1, b1, sc);
            continue;
          }
        }
        const uint4 wk = *reinterpret_cast<const uint4*>(Tq + (SPARSE ? 128 + 64 * (k - 1) : 64 * k));
        uint32_t op0[4], op1[4];
        fp8x4_to_bf16x4(wk.x, op0[0], op0[1]);
        fp8x4_to_bf16x4(wk.y, op0[2], op0[3]);
        fp8x4_to_bf16x4(wk.z, op1[0], op1[1]);
        fp8x4_to_bf16x4(wk.w, op1[2], op1[3]);
        const uint4 q0 = q_op(2 * k), q1 = q_op(2 * k + 1);
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

    // ROWS576: a tile's operands are staged in registers right after it lands (the QK chunks, the PV transposed reads,
    // the key scales), so its ring slot is refilled while it computes: all DEPTH slots of a wave are in flight then.
    // (bf16 rows compute from LDS: twice the operand registers would not fit beside the accumulators; sparse rows'
    // gathers are latency-bound, and staging measured slower there.)
    constexpr bool STAGED = FMT == ROWS576;
    constexpr int KST = SPARSE ? 10 : 9;  // 16-byte QK chunks per lane: ROWS640 has two rope chunks
    uint4 kst[STAGED ? KST : 1];
    uint2 vst[STAGED ? 16 : 1];
    float kss[4];
    auto stage = [&](const uint8_t* T, const uint8_t* S) {
      if constexpr (STAGED) {
        const uint8_t* Tq = T + key_of(li) * RS + 16 * g4;
        if constexpr (SPARSE) {
          kst[0] = *reinterpret_cast<const uint4*>(Tq);
          kst[1] = *reinterpret_cast<const uint4*>(Tq + 64);
#pragma unroll
          for (int k = 1; k < 9; ++k) kst[k + 1] = *reinterpret_cast<const uint4*>(Tq + 128 + 64 * (k - 1));
        } else {
          [[clang::always_inline]] load_chunks(T, RS, kst);
        }
        const uint8_t* Tv = T + key_of(4 * g4 + ((li >> 1) & 3)) * RS + (SPARSE ? 128 : 0) + 16 * (li >> 3) + 8 * (li & 1);
#pragma unroll
        for (int s = 0; s < 16; ++s) vst[s] = lds_read_tr8(Tv + 32 * s);
        [[clang::always_inline]] key_scales(S, kss);
      }
    };
    // scores and accumulate of the staged tile, as above
    auto scores_staged = [&](uint32_t vmask, float (&x)[4], float& tmax) {
      if constexpr (FP8QK) {
        const f32x4_t sc = qk_fp8(kst);
        tmax = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const bool ok = (vmask >> key_of(4 * g4 + r)) & 1u;
          x[r] = ok ? sc[r] * base_scale * kss[r] : -INFINITY;
          tmax = fmaxf(tmax, x[r]);
        }
        tmax = max_across_groups(tmax);
        return;
      }
      f32x4_t scp[3] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int k = 0; k < 9; ++k) {
        f32x4_t& sc = scp[k % 3];
        if constexpr (STAGED) {
          if (SPARSE && k == 0) {
            const uint32_t a0[4] = {kst[0].x, kst[0].y, kst[0].z, kst[0].w};
            const uint32_t a1[4] = {kst[1].x, kst[1].y, kst[1].z, kst[1].w};
            const uint4 q0 = q_op(0), q1 = q_op(1);
            const uint32_t b0[4] = {q0.x, q0.y, q0.z, q0.w}, b1[4] = {q1.x, q1.y, q1.z, q1.w};
            sc = mfma_16x16x32_bf16(a0, b0, sc);
            sc = mfma_16x16x32_bf16(a1, b1, sc);
            continue;
          }
          const uint4 wk = kst[SPARSE ? k + 1 : k];
          uint32_t op0[4], op1[4];
          fp8x4_to_bf16x4(wk.x, op0[0], op0[1]);
          fp8x4_to_bf16x4(wk.y, op0[2], op0[3]);
          fp8x4_to_bf16x4(wk.z, op1[0], op1[1]);
          fp8x4_to_bf16x4(wk.w, op1[2], op1[3]);
          const uint4 q0 = q_op(2 * k), q1 = q_op(2 * k + 1);
          const uint32_t b0[4] = {q0.x, q0.y, q0.z, q0.w}, b1[4] = {q1.x, q1.y, q1.z, q1.w};
          sc = mfma_16x16x32_bf16(op0, b0, sc);
          sc = mfma_16x16x32_bf16(op1, b1, sc);
        }
      }
      const f32x4_t sc = scp[0] + scp[1] + scp[2];
      tmax = -INFINITY;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool ok = (vmask >> key_of(4 * g4 + r)) & 1u;
        x[r] = ok ? sc[r] * base_scale * kss[r] : -INFINITY;
        tmax = fmaxf(tmax, x[r]);
      }
      tmax = max_across_groups(tmax);
    };
    auto accumulate_staged = [&](uint32_t vmask, const float (&x)[4]) {
      float pw[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool ok = (vmask >> key_of(4 * g4 + r)) & 1u;
        const float p = __builtin_amdgcn_exp2f(x[r] - m_ref);
        l_run += p;
        pw[r] = ok ? p * kss[r] : 0.0f;
      }
      const uint32_t pop[2] = {pack_bf16x2(pw[0], pw[1]), pack_bf16x2(pw[2], pw[3])};
      if constexpr (STAGED) {
#pragma unroll
        for (int s = 0; s < 16; ++s) {
          uint32_t op[2];
          fp8x4_to_bf16x4(vst[s].x, op[0], op[1]);
          acc[s >> 1][2 * (s & 1)] = mfma_16x16x16_bf16(op, pop, acc[s >> 1][2 * (s & 1)]);
          fp8x4_to_bf16x4(vst[s].y, op[0], op[1]);
          acc[s >> 1][2 * (s & 1) + 1] = mfma_16x16x16_bf16(op, pop, acc[s >> 1][2 * (s & 1) + 1]);
        }
      }
    };

    // ---- the tile loop: wave w takes tiles t_first + w + WAVES i through its ring of DEPTH slots; while one tile
    // computes, DEPTH (staged) or DEPTH - 1 tiles' loads are in flight ----
    {
      // VMEM operations one tile issues: its DMAs, plus the per-token scale DMA of the paged format
      constexpr int PER_TILE = NDMA + (FMT == ROWS576 ? 1 : 0);
      constexpr int AHEAD = STAGED ? DEPTH : DEPTH - 1;  // tiles issued before the loop
      static_assert(AHEAD * PER_TILE < 64, "vmcnt range");
      static_assert(AHEAD <= 4, "the waits below count at most three tiles");
      // wait until at most n tiles' loads (n <= 3) are in flight
      auto wait_tiles = [&](int32_t n) {
        if (n >= 3) wait_vmcnt<3 * PER_TILE>();
        else if (n == 2) wait_vmcnt<2 * PER_TILE>();
        else if (n == 1) wait_vmcnt<PER_TILE>();
        else wait_vmcnt<0>();
      };
      const int32_t t0 = t_first + wave;
      const int32_t mine = t0 < t_last ? (t_last - t0 + WAVES - 1) / WAVES : 0;
      const uint32_t ring = lds_address((lds_void*)(lds_u8*)&sm_ring[wave][0][0]);
      // The compiler's own loads (block table, query, indices) complete here, in a wait it sees (vmcnt(0): encoded
      // vmcnt 0, expcnt 7, lgkmcnt 15), before any DMA is in flight; otherwise it could wait for them again inside the
      // loop, and such a wait would drain the DMAs.
      __builtin_amdgcn_s_waitcnt(0x0f70);
      if constexpr (FP8QK) {
        // the query's 18 KB by 18 wave-wide DMAs dealt round-robin to the waves (a head past the group reads zeros)
        const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(a.ql + ((int64_t)b * a.H + 16 * hg) * kLatent), (short)0, nh * kLatent * 2, kBufferFlags);
        const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(a.qpe + ((int64_t)b * a.H + 16 * hg) * kRope), (short)0, nh * kRope * 2, kBufferFlags);
        const uint32_t qb = lds_address((lds_void*)(lds_u8*)&sm_qraw[0]);
        for (int k = wave; k < 18; k += WAVES) {
          if (k < 16) dma_buffer16(rq, qb + 1024 * k, 1024 * k + 16 * lane);
          else dma_buffer16(rr, qb + 1024 * k, 1024 * (k - 16) + 16 * lane);
        }
      }
#pragma unroll
      for (int i = 0; i < AHEAD; ++i)
        if (i < mine) issue(ring + i * SLOT, t0 + i * WAVES);
      if constexpr (FP8QK) {
        // this wave's query DMAs have landed (only its tiles' DMAs, issued after them, may be in flight), then every
        // wave's; lane (g4, li) takes its operand elements of head li
        static_assert(AHEAD == 2, "the waits below count two tiles");
        const int32_t n_after = min(mine, AHEAD);
        if (n_after >= 2) wait_vmcnt<2 * PER_TILE>();
        else if (n_after == 1) wait_vmcnt<PER_TILE>();
        else wait_vmcnt<0>();
        __syncthreads();
#pragma unroll
        for (int st = 0; st < 18; ++st) {
          const int off = st < 16 ? 1024 * li + 2 * (128 * (st >> 2) + 32 * g4 + 8 * (st & 3))
                                  : 16384 + 128 * li + 2 * (16 * g4 + 8 * (st & 1));
          qreg[st] = *reinterpret_cast<const uint4*>(&sm_qraw[off]);
        }
      }
      [[clang::always_inline]] split_query();
      // The own row, quantized as the store quantizes it, into sm_own in the pool's row format.
      if (own_wave) {
        const uint32_t wv[8] = {own0.x, own0.y, own0.z, own0.w, own1.x, own1.y, own1.z, own1.w};
        if constexpr (BF16) {
          // the row as it is: 72 16-byte chunks, lane l holding chunks l and 64 + l (l < 8)
          *reinterpret_cast<uint4*>(&sm_own[16 * lane]) = own0;
          if (lane < 8) *reinterpret_cast<uint4*>(&sm_own[16 * (lane + 64)]) = own1;
        } else if constexpr (FMT == ROWS576) {
          float m = 0.0f;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            m = fmaxf(m, fabsf(bf16_bits_to_f32(wv[j] & 0xffffu)));
            m = fmaxf(m, fabsf(bf16_bits_to_f32(wv[j] >> 16)));
          }
          own_s = scale_from_absmax(wave_max(m));
#pragma unroll
          for (int part = 0; part < 2; ++part) {
            if (part == 1 && lane >= 8) continue;
            uint32_t o[2] = {0, 0};
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              const uint32_t bits = (wv[part * 4 + (i >> 1)] >> ((i & 1) * 16)) & 0xffffu;
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
                const uint32_t lo = f32_to_bf16_bits(bf16_bits_to_f32(wv[part * 4 + i] & 0xffffu) / a.kv_scale);
                const uint32_t hi = f32_to_bf16_bits(bf16_bits_to_f32(wv[part * 4 + i] >> 16) / a.kv_scale);
                o[i] = lo | (hi << 16);
              }
              *reinterpret_cast<uint4*>(&sm_own[16 * ch]) = make_uint4(o[0], o[1], o[2], o[3]);
            } else {
#pragma unroll
              for (int i = 0; i < 8; ++i) {
                const uint32_t bits = (wv[part * 4 + (i >> 1)] >> ((i & 1) * 16)) & 0xffffu;
                sm_own[128 + latent_byte_of_dim(8 * (ch - 8) + i)] = (uint8_t)quantize_e4m3fn(bits, a.kv_scale);
              }
            }
          }
        }
      }
      // The own row's pool store, issued as soon as the row is packed. It sits among the DMAs, which only makes the
      // waits below stricter until it completes: a wait for tile i still needs fewer outstanding operations than the
      // DMAs issued after tile i, so tile i's have landed. (Issued after the tile loop, its completion fell on the
      // workgroup's tail: +1.2 µs on cfg3.) Paged formats; the sparse one stores its own row at the segment's end
      // (measured 0.2 µs better there, its unstaged ring being the more sensitive to a stricter wait).
      if (!SPARSE && own_wave && own_slot >= 0) {
        if constexpr (BF16) {
          uint8_t* dst = a.cache + own_slot * 1152;
          *reinterpret_cast<uint4*>(dst + 16 * lane) = own0;
          if (lane < 8) *reinterpret_cast<uint4*>(dst + 16 * (lane + 64)) = own1;
        } else if constexpr (FMT == ROWS576) {
  #pragma unroll
          for (int part = 0; part < 2; ++part) {
            if (part == 1 && lane >= 8) continue;
            *reinterpret_cast<uint2*>(a.cache + own_slot * 576 + 8 * (lane + 64 * part)) =
                make_uint2(own_q[2 * part], own_q[2 * part + 1]);
          }
          if (lane == 0) a.row_scale[own_slot] = own_s;
        } else {
          // the packed row is sm_own's first 640 bytes
          uint8_t* dst = a.cache + own_slot * 640;
          *reinterpret_cast<uint2*>(dst + 8 * lane) = *reinterpret_cast<const uint2*>(&sm_own[8 * lane]);
          if (lane < 16) *reinterpret_cast<uint2*>(dst + 512 + 8 * lane) = *reinterpret_cast<const uint2*>(&sm_own[512 + 8 * lane]);
        }
      }
      // The own row as key 0 of a one-key tile whose 16 rows all read sm_own (row stride 0; the other keys masked).
      if (own_wave) {
        float xo[4], to;
        [[clang::always_inline]] scores(&sm_own[0], 1u, xo, to, 0, &sm_own[kOwnScales]);
        if (needs_rescale(to)) [[clang::always_inline]] rescale(to);
        [[clang::always_inline]] accumulate(&sm_own[0], 1u, xo, 0, &sm_own[kOwnScales]);
      }
      // The rare rescale is a branch inside the loop, before the tile's PV. (Taken out of the loop, a tile that needed
      // it leaving the loop before its PV and re-entering after it, the compiler moved accumulator parts between the
      // VGPRs and AGPRs at every tile: 41.6 against 41.3 µs on cfg3, 20.1 against 19.4 on cfg5.)
      int slot = 0;
      float x[4], tmax = -INFINITY;
      uint32_t vm = 0;
      for (int32_t i = 0; i < mine; ++i) {
        uint8_t* T = &sm_ring[wave][slot][0];
        // wait until tile i's loads have landed (the loads of the tiles after it may stay in flight); unstaged, first
        // issue tile i + DEPTH - 1 into the slot tile i - 1 freed
        const int32_t ahead = mine - 1 - i;
        if constexpr (STAGED) {
          wait_tiles(min(ahead, DEPTH - 1));
        } else {
          if (ahead >= DEPTH - 1) {
            issue(ring + (slot == 0 ? DEPTH - 1 : slot - 1) * SLOT, t0 + (i + DEPTH - 1) * WAVES);
            wait_vmcnt<(DEPTH - 1) * PER_TILE>();
          } else if (ahead == 1) {
            wait_vmcnt<PER_TILE>();
          } else {
            wait_vmcnt<0>();
          }
        }
        vm = tile_mask(t0 + i * WAVES);
        if constexpr (SPARSE) {
          // rare: the gathers read a slot this launch stores an own row to (the loads drain first)
          if (const uint32_t al = (a.new_slots || a.spec > 1) ? tile_aliases(t0 + i * WAVES) : 0u) {
            wait_vmcnt<0>();
            patch_aliases(T, t0 + i * WAVES, al);
          }
        }
        if constexpr (STAGED) {
          if (vm != 0xffffu) [[clang::always_inline]] sanitize(T, vm);
          [[clang::always_inline]] stage(T, T + Geo::SCALES);
          [[clang::always_inline]] scores_staged(vm, x, tmax);
          // the staged reads have returned (QK has consumed its chunks): refill the slot with tile i + DEPTH
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          if (i + DEPTH < mine) issue(ring + slot * SLOT, t0 + (i + DEPTH) * WAVES);
        } else {
          [[clang::always_inline]] scores(T, vm, x, tmax, RS, T + Geo::SCALES);
        }
        if (needs_rescale(tmax)) [[clang::always_inline]] rescale(tmax);
        if constexpr (STAGED) [[clang::always_inline]] accumulate_staged(vm, x);
        else [[clang::always_inline]] accumulate(T, vm, x, RS, T + Geo::SCALES);
        slot = slot == DEPTH - 1 ? 0 : slot + 1;
      }
      wait_vmcnt<0>();
    }

    // ---- merge the waves: a common maximum per head; wave w sums latent blocks 2 w, 2 w + 1 over the waves ----
    const float l_w = sum_across_groups(l_run);
    if (g4 == 0) {
      sm_m[wave][li] = m_ref;
      sm_l[wave][li] = l_w;
    }
    __syncthreads();  // every wave is past its tile loop: the ring's space is free for the exchange
    float M = sm_m[0][li];
#pragma unroll
    for (int sw = 1; sw < WAVES; ++sw) M = fmaxf(M, sm_m[sw][li]);
    float L = 0.0f;
#pragma unroll
    for (int sw = 0; sw < WAVES; ++sw) L += __builtin_amdgcn_exp2f(sm_m[sw][li] - M) * sm_l[sw][li];
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
    const float oscale = SPARSE ? a.kv_scale : 1.0f;
    const int32_t pslot = 2 * w + (first_seg ? 0 : 1);
    const __amdgpu_buffer_rsrc_t ws_o_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)a.ws_o, (short)0, (int)(uint32_t)(2ll * a.n_ctas * a.H * kLatent * 4), kBufferFlags);
    const __amdgpu_buffer_rsrc_t ws_ml_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)a.ws_ml, (short)0, (int)(uint32_t)(2ll * a.n_ctas * a.H * 8), kBufferFlags);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      if (q / 2 != wave) continue;
      f32x4_t v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        v[r] = acc[q][r] * f;
#pragma unroll
        for (int sw = 0; sw < WAVES; ++sw) {
          if (sw == wave) continue;
          const int idx = q < 2 * sw ? q : q - 2;
          const float4 t = xchg(sw, idx)[r * 64 + lane];
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
      if (whole) {
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
        const int64_t prow = (int64_t)pslot * a.H + h;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          // partials are kept in latent-byte order (ROWS640: byte beta holds dim latent_dim_of_byte(beta)), so
          // each lane stores 16 bytes and a head's 4 lanes 64 contiguous bytes; the merge maps bytes to dims
          const int beta = 64 * q + 16 * r + 4 * g4;
          store_dev16(ws_o_rsrc, (uint32_t)((prow * kLatent + beta) * 4), make_float4(v[r][0], v[r][1], v[r][2], v[r][3]));
        }
        if (q == 0 && g4 == 0) store_dev8(ws_ml_rsrc, (uint32_t)(prow * 8), make_float2(M, L));
      }
    }

    // ---- a row split over workgroups: publish, count, and merge when the row is complete ----
    // The row's arrival word counts arrivals (bits 0 .. 15) and holds retracted blocks (bits 16 .. 23). The workgroup
    // that arrives k-th owns latent blocks c = k, k + n, ... (n = min(S, 8)). An owner polls, a bounded number of
    // times, until the count reaches S and merges its blocks; one whose polls run out retracts them (an atomic or of
    // their bits) unless the or finds every arrival counted, in which case it merges them itself. The last to arrive
    // merges its own blocks and those its add found retracted, and waits for nothing: each block is merged exactly once.
    // (A workgroup whose range goes on into another row retracts at once.)
    if (!whole) {
      const int32_t S = wb - wa + 1;
      const bool wa_second = cta_start(wa) != row_t0;          // the row is not wa's first segment
      const int32_t pair = b * a.groups + hg;
      int32_t* arrive = a.ws_cnt + kCounterStride * pair;
      wait_vmcnt<0>();  // this wave's partial stores are complete (written through) before the count
      __syncthreads();
      if (tid == 0) {
        const int32_t nown = min(S, 8);
        const int32_t old = __hip_atomic_fetch_add(arrive, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int32_t k = old & 0xffff;
        // a clean block counts the row's S arrivals 0 .. S - 1: anything else was left by an earlier launch (or one
        // overlapping this one on the workspace), and this row's merge cannot be trusted
        if (k >= S || ((uint32_t)old >> 24) != 0)
          __hip_atomic_fetch_or(a.ws_cnt + kStreamStatusWord, SNA_WS_DIRTY_ARRIVAL, __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT);
        uint32_t mine = 0;
        for (int32_t c = k; k < nown && c < 8; c += nown) mine |= 1u << c;
        uint32_t todo = 0;
        if (k == S - 1) {
          todo = mine | (((uint32_t)old >> 16) & 0xffu);
        } else if (mine) {
          int32_t seen = k + 1;
          // a workgroup with another segment after this one does not wait: the row's other pieces may be segments
          // that other workgroups reach only after their own merges, so its waits would chain across the launch
          const int32_t polls = s_hi < g_hi ? 0 : a.wait_polls;
          for (int32_t p = 0; seen < S && p < polls; ++p) {
            __builtin_amdgcn_s_sleep(1);
            seen = __hip_atomic_load(arrive, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & 0xffff;
          }
          if (seen >= S) {
            todo = mine;
          } else {
            const int32_t now = __hip_atomic_fetch_or(arrive, (int32_t)(mine << 16), __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_AGENT);
            if ((now & 0xffff) >= S) todo = mine;  // the last arrived before the or: it left these blocks here
          }
        }
        sm_word = (int32_t)todo;
      }
      __syncthreads();
      const uint32_t todo = (uint32_t)sm_word;
      static_assert(sizeof(sm_ring) >= 16 * 256 * sizeof(float2), "the merge's weights fit the ring");
      if (todo)
        merge_mask<SPARSE>(a, ws_o_rsrc, ws_ml_rsrc, b, hg, wa, wa_second, S, todo,
                           reinterpret_cast<float2*>(&sm_ring[0][0][0]));
      __syncthreads();
    }
    // ---- the sparse format's own row store (the paged formats store theirs before the tile loop); nothing in the
    // launch reads the slot: a gather of it takes the packed source row ----
    if (SPARSE && own_wave && own_slot >= 0) {
      // the packed row is sm_own's first 640 bytes
      uint8_t* dst = a.cache + own_slot * 640;
      *reinterpret_cast<uint2*>(dst + 8 * lane) = *reinterpret_cast<const uint2*>(&sm_own[8 * lane]);
      if (lane < 16) *reinterpret_cast<uint2*>(dst + 512 + 8 * lane) = *reinterpret_cast<const uint2*>(&sm_own[512 + 8 * lane]);
    }
    g = s_hi;
    row_t0 = row_t1;
    if constexpr (!MULTI) break;
    __syncthreads();  // every wave is done with the ring's merge exchange before the next segment refills the ring
  }

  // ---- the launch's last workgroup returns the counters to zero (every other one has finished with them: its
  // atomics on them have returned; its output stores need not have landed, so none is waited for here) ----
  __syncthreads();
  if (tid == 0) {
    const int32_t done = __hip_atomic_fetch_add(a.ws_cnt + kStreamDoneWord, 1, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
    if (done < 0 || done >= (int32_t)(gridDim.x * gridDim.y))
      __hip_atomic_fetch_or(a.ws_cnt + kStreamStatusWord, SNA_WS_DIRTY_DONE, __ATOMIC_RELAXED,
                            __HIP_MEMORY_SCOPE_AGENT);
    sm_word = done == (int32_t)(gridDim.x * gridDim.y) - 1;
  }
  __syncthreads();
  if (sm_word) {
    for (int32_t i = tid; i < a.B * a.groups; i += NT)
      __hip_atomic_store(a.ws_cnt + kCounterStride * i, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (tid == 0) __hip_atomic_store(a.ws_cnt + kStreamDoneWord, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

static int check_plan(const sna_split_plan* plan, int32_t B, int32_t groups, const char* what, bool* multi) {
  if (!plan || plan->tile != 16 || plan->batch != B || plan->n_ctas < 0 || plan->n_ctas > SNA_MAX_CTAS)
    return fail(SNA_ERR_INVALID_ARGUMENT, "%s: missing or foreign split plan (made for %d rows)", what,
                plan ? plan->batch : -1);
  if (B > SNA_MAX_PLAN_ROWS || (int64_t)B * groups > kStreamMaxCounters)
    return fail(SNA_ERR_UNSUPPORTED, "%s: %d rows x %d head groups exceed the stream split's counters", what, B, groups);
  // the stream split must cover every row's tiles in increasing order, as the kernel walks it
  int64_t total = 0;
  for (int32_t b = 0; b < B; ++b) {
    if (plan->row_keys[b] < 0) return fail(SNA_ERR_INVALID_ARGUMENT, "%s: plan row %d has negative keys", what, b);
    total += std::max((plan->row_keys[b] + 15) / 16, 1);
  }
  if (total != plan->total_tiles || (B > 0 && plan->n_ctas < 1) || plan->cta_start[0] != 0 ||
      (int64_t)plan->cta_start[plan->n_ctas] != total)
    return fail(SNA_ERR_INVALID_ARGUMENT, "%s: the plan's stream split does not cover its rows' %lld tiles", what,
                (long long)total);
  for (int32_t w = 0; w < plan->n_ctas; ++w) {
    if (plan->cta_start[w + 1] <= plan->cta_start[w] || plan->cta_row[w] >= B)
      return fail(SNA_ERR_INVALID_ARGUMENT, "%s: plan workgroup %d has an empty range or a row past %d", what, w, B);
    int64_t first = 0;
    for (int32_t b = 0; b < plan->cta_row[w]; ++b) first += std::max((plan->row_keys[b] + 15) / 16, 1);
    const int64_t last = first + std::max((plan->row_keys[plan->cta_row[w]] + 15) / 16, 1);
    if ((int64_t)plan->cta_start[w] != first + plan->cta_off[w] || (int64_t)plan->cta_start[w] >= last)
      return fail(SNA_ERR_INVALID_ARGUMENT, "%s: plan workgroup %d does not start at its row's tile", what, w);
    if ((int64_t)plan->cta_start[w + 1] > last) *multi = true;
  }
  return SNA_OK;
}

static void fill_stream_args(MlaArgs& a, const sna_split_plan* plan, float* ws) {
  a.n_ctas = plan->n_ctas;
  a.wait_polls = plan->wait_polls;
  a.ws_cnt = (int32_t*)ws;
  a.ws_o = (float*)((uint8_t*)ws + kStreamCounterBytes);
  a.ws_ml = a.ws_o + 2ll * plan->n_ctas * a.H * kLatent;
  for (int32_t w = 0; w <= plan->n_ctas; ++w) a.cta_start[w] = plan->cta_start[w];
  for (int32_t w = 0; w < plan->n_ctas; ++w) {
    a.cta_row_off[w] = (uint32_t)plan->cta_row[w] << 16 | plan->cta_off[w];
  }
  if (!plan->device_split)
    for (int32_t b = 0; b < plan->batch; ++b) a.row_keys[b] = plan->row_keys[b];
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
  if (cache_dtype != SNA_DTYPE_FP8_E4M3FN && cache_dtype != SNA_DTYPE_BF16)
    return fail(SNA_ERR_INVALID_ARGUMENT, "mla_decode: unknown cache dtype %d", cache_dtype);
  const bool bf16 = cache_dtype == SNA_DTYPE_BF16;
  if (B < 0 || num_heads < 1 || page_size < 16 || page_size % 16 || num_blocks < 1 || table_width < 0 ||
      table_stride < table_width || !(sm_scale > 0.0f) || num_blocks * page_size > INT32_MAX)
    return fail(SNA_ERR_INVALID_ARGUMENT, "mla_decode: bad sizes (B %d, heads %d, page %d (a multiple of 16), blocks "
                "%lld, table %d/%lld)", B, num_heads, page_size, (long long)num_blocks, table_width,
                (long long)table_stride);
  const int32_t groups = (num_heads + 15) / 16;
  bool multi = false;
  const bool dev = plan && plan->device_split;
  if (dev) {
    // a plan from a bound: the launch cuts its stream from the device's seq_lens; whole rows when every row can have
    // a workgroup, equal ranges across rows otherwise
    if (plan->tile != 16 || plan->batch != B || plan->n_ctas < 1 || plan->n_ctas > SNA_MAX_CTAS)
      return fail(SNA_ERR_INVALID_ARGUMENT, "mla_decode: missing or foreign split plan (made for %d rows)", plan->batch);
    if (B > SNA_MAX_PLAN_ROWS || (int64_t)B * groups > kStreamMaxCounters)
      return fail(SNA_ERR_UNSUPPORTED, "mla_decode: %d rows x %d head groups exceed the stream split's counters", B,
                  groups);
    multi = B > plan->n_ctas;
  } else if (int rc = check_plan(plan, B, groups, "mla_decode", &multi)) {
    return rc;
  }
  if (B == 0) return SNA_OK;
  const int64_t need = sna_decode_workspace_bytes(plan, num_heads, kLatent);
  if (!ql_nope || !q_pe || !cache || (!bf16 && !row_scale) || !block_table || !compact_new || !out || !workspace ||
      (dev && !seq_lens))
    return fail(SNA_ERR_INVALID_ARGUMENT, "mla_decode: null pointer");
  if (!aligned(ql_nope, 16) || !aligned(q_pe, 16) || !aligned(cache, 16) || !aligned(compact_new, 16) ||
      (!bf16 && !aligned(row_scale, 16)) || !aligned(workspace, 256))
    return fail(SNA_ERR_INVALID_ARGUMENT, "mla_decode: q, cache and row_scale must be 16-byte aligned, the workspace "
                "256-byte aligned");
  if (workspace_bytes < need)
    return fail(SNA_ERR_WORKSPACE, "mla_decode: workspace of %lld bytes, the plan needs %lld",
                (long long)workspace_bytes, (long long)need);
  MlaArgs a{};
  a.ql = (const uint16_t*)ql_nope;
  a.qpe = (const uint16_t*)q_pe;
  a.cache = (uint8_t*)cache;
  a.row_scale = (float*)row_scale;
  a.kv_scale = 1.0f;
  a.table = block_table;
  a.table_stride = table_stride;
  a.table_width = table_width;
  a.own = (const uint16_t*)compact_new;
  a.new_slots = new_slots;
  a.spec = 1;
  a.B = B;
  a.H = num_heads;
  a.P = page_size;
  a.groups = groups;
  a.num_blocks = num_blocks;
  a.sm_scale = sm_scale;
  a.out = (uint16_t*)out;
  a.lse_out = nullptr;
  a.seq_lens = seq_lens;  // read by a device-split launch only: an exact plan's host lengths drive the others
  fill_stream_args(a, plan, (float*)workspace);
  const dim3 grid(plan->n_ctas, groups);
  hipStream_t s = (hipStream_t)stream;
#define SNA_MLA_LAUNCH(F, M, D) hipLaunchKernelGGL((mla_decode_kernel<F, false, M, D>), grid, dim3(256), 0, s, a)
  if (bf16) {
    if (dev) { if (multi) SNA_MLA_LAUNCH(ROWS1152, true, true); else SNA_MLA_LAUNCH(ROWS1152, false, true); }
    else if (multi) SNA_MLA_LAUNCH(ROWS1152, true, false);
    else SNA_MLA_LAUNCH(ROWS1152, false, false);
  } else {
    if (dev) { if (multi) SNA_MLA_LAUNCH(ROWS576, true, true); else SNA_MLA_LAUNCH(ROWS576, false, true); }
    else if (multi) SNA_MLA_LAUNCH(ROWS576, true, false);
    else SNA_MLA_LAUNCH(ROWS576, false, false);
  }
#undef SNA_MLA_LAUNCH
  return check_launch("mla_decode");
}

extern "C" int sna_mla_decode_sparse(const void* q_absorbed, const void* q_pe, const void* cache, float kv_scale,
                                     const int32_t* indices, int32_t n_indices, const int32_t* block_table,
                                     int64_t table_stride, int32_t table_width, const int32_t* positions,
                                     const void* own_rows, const int64_t* new_slots, float sm_scale, void* ctx_out,
                                     float* lse_out, int32_t B, int32_t spec,
                                     int32_t num_heads, int32_t page_size, int64_t num_blocks,
                                     const sna_split_plan* plan, void* workspace, int64_t workspace_bytes,
                                     void* stream) {
  ApiGuard guard;
  if (B < 0 || num_heads < 1 || n_indices < 0 || page_size < 1 || num_blocks < 1 || table_width < 0 ||
      table_stride < table_width || !(sm_scale > 0.0f) || !(kv_scale > 0.0f) || num_blocks * page_size > INT32_MAX)
    return fail(SNA_ERR_INVALID_ARGUMENT, "mla_decode_sparse: bad sizes (B %d, heads %d, indices %d, page %d, blocks "
                "%lld, table %d/%lld, kv_scale %g)", B, num_heads, n_indices, page_size, (long long)num_blocks,
                table_width, (long long)table_stride, (double)kv_scale);
  if (spec < 1 || B % spec)
    return fail(SNA_ERR_INVALID_ARGUMENT, "mla_decode_sparse: %d query tokens are not whole sequences of spec %d", B,
                spec);
  const int32_t row_keys = n_indices + spec - 1;  // the index list, then the spec - 1 siblings' own rows
  const int32_t groups = (num_heads + 15) / 16;
  bool multi = false;
  if (plan && plan->device_split)
    return fail(SNA_ERR_INVALID_ARGUMENT, "mla_decode_sparse: a sparse plan is exact (its rows' key counts are the "
                "index list's length); a device-split plan is for the paged MLA decode");
  if (int rc = check_plan(plan, B, groups, "mla_decode_sparse", &multi)) return rc;
  if (B == 0) return SNA_OK;
  for (int32_t b = 0; b < B; ++b)
    if (plan->row_keys[b] != row_keys)
      return fail(SNA_ERR_INVALID_ARGUMENT, "mla_decode_sparse: the plan was made for %d keys per row, not %d (%d "
                  "indices and %d siblings)", plan->row_keys[b], row_keys, n_indices, spec - 1);
  for (int32_t w = 0; w < plan->n_ctas; ++w)
    if (plan->cta_start[w + 1] - plan->cta_start[w] > (uint32_t)(kMlaMaxSplitKeys / 16))
      return fail(SNA_ERR_INVALID_ARGUMENT, "mla_decode_sparse: plan workgroup %d holds more than %d index tiles", w,
                  kMlaMaxSplitKeys / 16);
  const int64_t need = sna_decode_workspace_bytes(plan, num_heads, kLatent);
  if (!q_absorbed || !q_pe || !cache || !block_table || !positions || !own_rows || !ctx_out ||
      (n_indices > 0 && !indices) || !workspace)
    return fail(SNA_ERR_INVALID_ARGUMENT, "mla_decode_sparse: null pointer");
  if (!aligned(q_absorbed, 16) || !aligned(q_pe, 16) || !aligned(cache, 16) || !aligned(workspace, 256))
    return fail(SNA_ERR_INVALID_ARGUMENT, "mla_decode_sparse: q and cache must be 16-byte aligned, the workspace "
                "256-byte aligned");
  if (workspace_bytes < need)
    return fail(SNA_ERR_WORKSPACE, "mla_decode_sparse: workspace of %lld bytes, the plan needs %lld",
                (long long)workspace_bytes, (long long)need);
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
  a.spec = spec;
  a.positions = positions;
  a.own = (const uint16_t*)own_rows;
  a.new_slots = new_slots;
  a.B = B;
  a.H = num_heads;
  a.P = page_size;
  a.groups = groups;
  a.num_blocks = num_blocks;
  a.sm_scale = sm_scale;
  a.out = (uint16_t*)ctx_out;
  a.lse_out = lse_out;
  fill_stream_args(a, plan, (float*)workspace);
  const bool wide = num_blocks * page_size * (int64_t)RowFmt<ROWS640>::kRowBytes > 0xffffffffll;
  const dim3 grid(plan->n_ctas, groups);
  hipStream_t s = (hipStream_t)stream;
#define SNA_DSA_LAUNCH(W, M)                                                                                  \
  do {                                                                                                        \
    if (spec > 1) hipLaunchKernelGGL((mla_decode_kernel<ROWS640, W, M, false, true>), grid, dim3(256), 0, s, a); \
    else hipLaunchKernelGGL((mla_decode_kernel<ROWS640, W, M>), grid, dim3(256), 0, s, a);                     \
  } while (0)
  if (wide) {
    if (multi) SNA_DSA_LAUNCH(true, true);
    else SNA_DSA_LAUNCH(true, false);
  } else {
    if (multi) SNA_DSA_LAUNCH(false, true);
    else SNA_DSA_LAUNCH(false, false);
  }
#undef SNA_DSA_LAUNCH
  return check_launch("mla_decode_sparse");
}

namespace {
__global__ __launch_bounds__(256) void zero_words_kernel(int32_t* p, int32_t n) {
  for (int32_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) p[i] = 0;
}
}  // namespace

extern "C" int sna_stream_workspace_status(void* workspace, int64_t workspace_bytes, int32_t* status, void* stream) {
  ApiGuard guard;
  if (!workspace || !status || workspace_bytes < kStreamCounterBytes)
    return fail(SNA_ERR_INVALID_ARGUMENT, "stream_workspace_status: null pointer or a workspace of %lld bytes "
                "(the counter block is %lld)", (long long)workspace_bytes, (long long)kStreamCounterBytes);
  hipStream_t s = (hipStream_t)stream;
  int32_t* word = (int32_t*)workspace + kStreamStatusWord;
  int32_t v = 0;
  static const int32_t zero = 0;
  if (hipMemcpyAsync(&v, word, sizeof(v), hipMemcpyDeviceToHost, s) != hipSuccess || hipStreamSynchronize(s) != hipSuccess)
    return fail(SNA_ERR_LAUNCH, "stream_workspace_status: reading the status word failed: %s",
                hipGetErrorString(hipGetLastError()));
  if (v != 0 && (hipMemcpyAsync(word, &zero, sizeof(zero), hipMemcpyHostToDevice, s) != hipSuccess ||
                 hipStreamSynchronize(s) != hipSuccess))
    return fail(SNA_ERR_LAUNCH, "stream_workspace_status: clearing the status word failed: %s",
                hipGetErrorString(hipGetLastError()));
  *status = v;
  return SNA_OK;
}

extern "C" int sna_stream_workspace_reset(void* workspace, int64_t workspace_bytes, void* stream) {
  ApiGuard guard;
  if (!workspace || workspace_bytes < kStreamCounterBytes)
    return fail(SNA_ERR_INVALID_ARGUMENT, "stream_workspace_reset: null pointer or a workspace of %lld bytes "
                "(the counter block is %lld)", (long long)workspace_bytes, (long long)kStreamCounterBytes);
  const int32_t n = (int32_t)(kStreamCounterBytes / 4);
  hipLaunchKernelGGL(zero_words_kernel, dim3(64), dim3(256), 0, (hipStream_t)stream, (int32_t*)workspace, n);
  return check_launch("stream_workspace_reset");
}
