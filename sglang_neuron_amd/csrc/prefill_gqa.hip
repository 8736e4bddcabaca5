// Segmented prefill attention over the paged pool (GQA, FP8 K/V with per-KV-head scales): a chunk's queries attend
// to their request's prior and, causally, to the chunk itself, all read from the pool (the chunk's K/V are stored
// before the attention runs), optionally inside a sliding window and with a sink logit per head.
//   reference: segmented_attention / _torch_segmented_attention (ops/attention/attention_segmented_cte.py:21-75)
//
// Work: one workgroup of 4 waves per (request, block of query tokens, KV head), dealt to the XCDs in contiguous runs
// so the blocks that read one request's keys of a KV head share an L2 (the DMAs keep the default cache policy for
// those rereads). Its 128 query rows are (token, head)
// pairs, token-major (row = t * group + j for the group's query head j); wave w owns rows 32 w .. 32 w + 31 as two
// 16-row MFMA N tiles. Keys run in tiles of 64 positions (FP8; 32 for bf16 pools) from the window's first key to
// the block's last query, each tile NSUB sub-tiles of 32 keys. A tile's K and V rows are DMA'd into a 2-slot LDS
// ring shared by the 4 waves (each wave issues a share of the tile's DMAs); one tile loads while one computes. The
// block-table entries of the key range are staged in LDS first, and a tile's four 16-key groups' byte offsets are
// computed by four lanes from one LDS round trip (lane reads hand them to the DMAs).
//
// Lane roles (lane = 16 g4 + i), per 32-key sub-tile:
//   QK  S^T[key, row] = K[key, :] . Q[row, :] per 16-key half a: lane (g4, i) feeds key 8 (i / 4) + 4 a + i % 4.
//       FP8: its bytes 32 g4 .. + 31 straight from LDS into v_mfma_scale_f32_16x16x128_f8f6f4 against the query's
//       two exact e4m3fn parts (below); bf16: elements 32 s + 8 g4 .. + 7 per step s into v_mfma_f32_16x16x32_bf16.
//       The result hands lane (g4, i) keys 8 g4 + 4 a + r (r < 4) of row i: over both halves the 8 consecutive keys
//       8 g4 .. 8 g4 + 7.
//   PV  O^T[dim, row] += V^T[dim, key] . P^T[key, row] per 16-dim tile c (v_mfma_f32_16x16x32_bf16): lane (g4, i)
//       supplies P^T for keys 8 g4 .. + 7 of row i (its own probabilities) and V^T's bf16 values of those keys at
//       dim 16 c + i: FP8, one ds_read_b64_tr_b8 of the ring's V rows converted in registers; bf16, from a V^T the
//       4 waves build once per tile in LDS.
//   acc lane (g4, i) holds row i at dims 16 c + 4 g4 + r.
// Online softmax in the log2 domain with a lazily moved reference maximum (as the decode kernels). Keys that no row
// of the block may see (past the chunk, or on an invalid page) have their V bytes zeroed in registers, so stale
// pool bytes cannot reach the output through p = 0.

#include "sna_device.h"
#include "sna_host.h"

namespace sna {

struct PrefillArgs {
  const uint16_t* q;       // [T, H, D] bf16
  const uint8_t* k_cache;  // [num_blocks, G, P, D] e4m3fn
  const uint8_t* v_cache;
  const float* k_scale;  // [G] dequantization scales, or (mul_scale) GPT-OSS multipliers m: a byte is worth byte / m
  const float* v_scale;
  bool mul_scale;
  const int32_t* table;  // [R, table_width] (row stride table_stride)
  int64_t table_stride;
  int32_t table_width;
  const int32_t* q_start;  // [R + 1] the requests' first rows in q
  const int32_t* prior;    // [R] prior tokens of each request
  const float* sinks;      // [H] natural-log sink logits, or null
  uint16_t* out;           // [T, H, D] bf16
  int32_t R, H, G, P, group, bq;  // bq: query tokens per workgroup (128 / group)
  int64_t num_blocks;
  float sm_scale;
  int32_t window;
};

template <int D, int ESZ>  // ESZ: bytes per K/V element (1: e4m3fn, 2: bf16)
struct PrefillGeo {
  static constexpr int TK = ESZ == 1 ? 64 : 32;              // keys per tile: NSUB sub-tiles of 32
  static constexpr int NSUB = TK / 32;
  static constexpr int ROWB = D * ESZ;                       // bytes of a K or V row
  static constexpr int CH = ROWB / 16;                       // 16-byte chunks of a K or V row
  static constexpr int STRIDE = CH + 1;                      // plus a pad chunk
  static constexpr int RS = 16 * STRIDE;                     // LDS row stride, bytes
  static constexpr int HALF = TK * RS;                       // the K (or V) rows of a tile
  static constexpr int SLOT = 2 * HALF;                      // one ring slot: K then V
  static constexpr int NDMA = (TK * STRIDE + 63) / 64;       // wave-wide DMAs of one of K, V
  static constexpr int TAIL = TK * STRIDE - 64 * (NDMA - 1);  // active lanes of the last one
  static constexpr int NI = 2 * NDMA;                        // DMAs of a tile, dealt round-robin to the 4 waves
  static constexpr int CNT_HI = (NI + 3) / 4, CNT_LO = NI / 4;  // a wave's DMAs per tile (waves < NI % 4: CNT_HI)
  static constexpr int DEPTH = 2;                            // the ring: one tile loads while one computes
  static constexpr int VT_RS = 2 * TK + 16;                  // bf16 V^T: a dim's TK keys, padded
  static constexpr int PAGES = 2048;  // block-table entries staged in LDS at a time
};

constexpr float kPrefillRescaleSlack = 8.0f;
constexpr int kPrefillBufferFlags = 0x00020000;  // dword 3 of a raw buffer resource (gfx9 family)

// BUF: each cache is under 4 GiB, so its tiles load through a buffer resource (the page base a uniform SGPR offset);
// otherwise through 64-bit addresses. The buffer forms of head dim 64 and of bf16 pools fit three workgroups' waves
// per SIMD (at most 168 VGPRs, no spill); the others take two.
template <int D, bool BUF, int ESZ>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu((BUF && (D == 64 || ESZ == 2)) ? 3 : 2)))
void prefill_gqa_kernel(PrefillArgs a) {
  using Geo = PrefillGeo<D, ESZ>;
  constexpr int ROWB = Geo::ROWB;
  constexpr int CH = Geo::CH, STRIDE = Geo::STRIDE, RS = Geo::RS, HALF = Geo::HALF, SLOT = Geo::SLOT;
  constexpr int NDMA = Geo::NDMA, NI = Geo::NI, DEPTH = Geo::DEPTH, TK = Geo::TK, NSUB = Geo::NSUB;
  constexpr int NS = D / 32;  // QK steps
  constexpr int NC = D / 16;  // PV dim tiles
  typedef __attribute__((address_space(3))) void lds_void;
  typedef __attribute__((address_space(3))) uint8_t lds_u8;
  __shared__ __attribute__((aligned(16))) uint8_t sm_ring[DEPTH * SLOT];
  __shared__ int32_t sm_pages[Geo::PAGES];
  // bf16 pools: the current tile's V, transposed once (each wave a quarter): row d holds the TK keys' values.
  __shared__ __attribute__((aligned(16))) uint8_t sm_vt[D * Geo::VT_RS];

  const int tid = threadIdx.x, lane = tid & 63, g4 = lane >> 4, li = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // XCD-aware order: each XCD takes a contiguous run of the (query block, request, KV head) order, so the query
  // blocks that read the same request's keys of one KV head share that XCD's L2
  const uint32_t lin = xcd_order(blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z),
                                 gridDim.x * gridDim.y * gridDim.z);
  const int32_t bx = (int32_t)(lin % gridDim.x);
  const int32_t r = (int32_t)((lin / gridDim.x) % gridDim.y), g = (int32_t)(lin / (gridDim.x * gridDim.y));
  const int32_t qa = a.q_start[r];
  const int32_t S = a.q_start[r + 1] - qa;
  const int32_t nqb = (S + a.bq - 1) / a.bq;
  if (bx >= nqb) return;
  const int32_t q0 = (nqb - 1 - bx) * a.bq;  // the blocks with the most keys start first
  const int32_t nq = min(a.bq, S - q0);
  const int32_t pos0 = a.prior[r] + q0;  // position of the block's first query
  const int32_t hi = pos0 + nq;          // the block reads keys [lo, hi)
  const int32_t lo = a.window > 0 ? max(0, pos0 - a.window + 1) : 0;

  // ---- this lane's two rows (N tiles n = 0, 1): token, head, position, and the query operand ----
  int32_t tok[2], head[2], qpos[2];
  bool row_ok[2];
  // The query operand of the FP8 QK: lane (g4, i) supplies dims 32 g4 .. 32 g4 + 31 of row i (zeros past d), the bf16
  // values scaled by a power of two sc (the row's absolute maximum into [128, 256)) and split exactly into two e4m3fn
  // parts, hi + lo / 16 (hi keeps the top 4 significant bits, lo the next 4). The MFMA's per-lane E8M0 B scales
  // undo sc (and the 1/16 of lo), so K . Q is the exact bf16 dot product accumulated in fp32.
  // A bf16 pool instead takes the bf16 query elements 32 s + 8 g4 .. + 7 for v_mfma_f32_16x16x32_bf16 (qf).
  uint32_t qhi[2][8], qlo[2][8];
  int32_t qsc_hi[2], qsc_lo[2];
  uint32_t qf[2][ESZ == 2 ? NS : 1][4];
#pragma unroll
  for (int n = 0; n < 2; ++n) {
    const int32_t row = 32 * wave + 16 * n + li;
    int32_t t = row / a.group;
    row_ok[n] = t < nq;
    t = min(t, nq - 1);  // a row past the block computes as its last token and is not written
    tok[n] = qa + q0 + t;
    head[n] = g * a.group + row % a.group;
    qpos[n] = pos0 + t;
    if constexpr (ESZ == 2) {
      const uint16_t* qb = a.q + ((int64_t)tok[n] * a.H + head[n]) * D + 8 * g4;
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const uint4 w = ld16(qb + 32 * s);
        qf[n][s][0] = w.x, qf[n][s][1] = w.y, qf[n][s][2] = w.z, qf[n][s][3] = w.w;
      }
      continue;
    }
    float v[32];
    const bool mine = 32 * g4 < D;
    const uint16_t* qp = a.q + ((int64_t)tok[n] * a.H + head[n]) * D + (mine ? 32 * g4 : 0);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint4 w = mine ? ld16(qp + 8 * c) : make_uint4(0, 0, 0, 0);
      const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[8 * c + 2 * e] = bf16_bits_to_f32(ww[e] & 0xffffu);
        v[8 * c + 2 * e + 1] = bf16_bits_to_f32(ww[e] >> 16);
      }
    }
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 32; ++e) amax = fmaxf(amax, fabsf(v[e]));
    amax = max_across_groups(amax);
    // sc = 2^(7 - floor(log2 amax)): amax * sc in [128, 256); E8M0 scale of hi = 127 - log2 sc, of lo 4 less
    // (the exponent is held to [-116, 127], where sc and both E8M0 scales are representable; a row that small only
    // loses bits far below the tolerance)
    const int32_t ex = amax > 0.0f ? max((int32_t)((__float_as_uint(amax) >> 23) & 0xff) - 127, -116) : -7;
    const float sc = __uint_as_float((uint32_t)(127 + 7 - ex) << 23);
    qsc_hi[n] = 127 + ex - 7;
    qsc_lo[n] = 127 + ex - 7 - 4;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      float h4[4], l4[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) split_q(v[4 * k + e] * sc, h4[e], l4[e]);
      qhi[n][k] = pack_e4m3fn_x4(h4[0], h4[1], h4[2], h4[3]);
      qlo[n][k] = pack_e4m3fn_x4(l4[0], l4[1], l4[2], l4[3]);
    }
  }
  const float k_deq = ESZ == 1 ? (a.mul_scale ? 1.0f / a.k_scale[g] : a.k_scale[g]) : 1.0f;
  const float qk_scale = a.sm_scale * kLog2e * k_deq;
  const float v_scale = ESZ == 1 ? (a.mul_scale ? 1.0f / a.v_scale[g] : a.v_scale[g]) : 1.0f;

  float m_ref[2] = {kNegBig, kNegBig}, l_run[2] = {0.0f, 0.0f};
  f32x4_t acc[2][NC];
#pragma unroll
  for (int n = 0; n < 2; ++n)
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[n][c] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // Each lane's LDS chunk o = 64 jj + lane of DMA jj (of K or V): chunk o % STRIDE of tile row o / STRIDE (the pad
  // chunk repeats the row's last chunk; lanes past the tile only occur in the last DMA, which switches them off).
  const uint32_t ring = lds_address((lds_void*)(lds_u8*)&sm_ring[0]);
  const int64_t head_stride = (int64_t)a.P * ROWB;  // bytes between KV heads of one page

  int32_t p0 = 0;  // first page index staged in sm_pages
  const bool p_pow2 = (a.P & (a.P - 1)) == 0;  // uniform: the page column of a key is a shift
  const int p_shift = __builtin_ctz((uint32_t)a.P);
  // This wave's DMAs of a tile: the m-th is DMA j = wave + 4 m of the tile (K for j < NDMA, then V), whose 64 lanes
  // fill LDS chunks 64 jj .. 64 jj + 63 of the K or V rows. Its rows span at most two 16-key groups (glo and glo + 1;
  // a group lies in one page): per lane, the byte offset inside the group and whether the lane's row is in glo + 1.
  // (lanes past the tile, only in a tile's last DMA when TAIL < 64, are switched off: bit 30 of dma_pk)
  constexpr int MW = Geo::CNT_HI;
  const int cnt = (wave < NI % 4 || NI % 4 == 0) ? Geo::CNT_HI : Geo::CNT_LO;
  uint32_t dma_pk[MW];   // offset in the group | (lane off) << 30 | (lane's row in group glo + 1) << 31
  int32_t dma_glo[MW];   // uniform
  uint32_t dma_lds[MW];  // uniform LDS offset in the slot
#pragma unroll
  for (int m = 0; m < MW; ++m) {
    const int j = min(wave + 4 * m, NI - 1);
    const int jj = j < NDMA ? j : j - NDMA;
    const int o = 64 * jj + lane;
    const int row = o / STRIDE, c = min(o % STRIDE, CH - 1);
    const int glo = (64 * jj / STRIDE) >> 4;
    dma_glo[m] = glo;
    const bool off = jj == NDMA - 1 && lane >= Geo::TAIL;
    dma_pk[m] = (uint32_t)((row & 15) * ROWB + 16 * c) | ((uint32_t)off << 30) | ((uint32_t)((row >> 4) > glo) << 31);
    dma_lds[m] = (j < NDMA ? 0 : HALF) + 1024 * jj;
  }
  const int64_t cache_bytes = a.num_blocks * a.G * head_stride;
  const __amdgpu_buffer_rsrc_t k_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)a.k_cache, (short)0, BUF ? (int)(uint32_t)cache_bytes : 0, kPrefillBufferFlags);
  const __amdgpu_buffer_rsrc_t v_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)a.v_cache, (short)0, BUF ? (int)(uint32_t)cache_bytes : 0, kPrefillBufferFlags);
  // Tile t's DMAs, and its pages' validity (bit u: the page of keys TK t + 16 u .. + 15 is valid; uniform), which
  // the tile's compute takes. Lane u (lanes past the tile's groups repeat its last, the spare a DMA whose rows end
  // in the last group reads) looks up its 16-key group's page and computes the group's byte offset, so the tile's
  // page lookups are one LDS round trip and its address arithmetic vector work; each DMA reads its two groups'
  // offsets with lane reads.
  auto issue = [&](int32_t t, int slot) -> uint32_t {
    const int32_t key = TK * t + 16 * min(lane, TK / 16 - 1);
    const int32_t col = p_pow2 ? key >> p_shift : key / a.P;
    const int32_t pg = sm_pages[col - p0];  // -1: invalid
    const int64_t goff = ((int64_t)max(pg, 0) * a.G + g) * head_stride + (int64_t)(key - col * a.P) * ROWB;
    const uint32_t pg_ok = (uint32_t)__ballot(pg >= 0) & ((1u << (TK / 16)) - 1u);
#pragma unroll
    for (int m = 0; m < MW; ++m) {
      if (m >= cnt) break;
      const int j = wave + 4 * m;
      const uint32_t lds = ring + slot * SLOT + dma_lds[m];
      if (Geo::TAIL < 64 && (dma_pk[m] >> 30 & 1u)) continue;
      if constexpr (BUF) {  // offsets < 4 GiB
        const uint32_t blo = __builtin_amdgcn_readlane((uint32_t)goff, dma_glo[m]);
        const uint32_t bhi = __builtin_amdgcn_readlane((uint32_t)goff, dma_glo[m] + 1);
        const uint32_t voff = ((dma_pk[m] >> 31) ? bhi : blo) + (dma_pk[m] & 0x3fffffffu);
        dma_buffer16_cached(j < NDMA ? k_rsrc : v_rsrc, lds, voff);
      } else {
        const int64_t blo = readlane_i64(goff, dma_glo[m]), bhi = readlane_i64(goff, dma_glo[m] + 1);
        const int64_t off = ((dma_pk[m] >> 31) ? bhi : blo) + (int64_t)(dma_pk[m] & 0x3fffffffu);
        dma_global16_cached((j < NDMA ? a.k_cache : a.v_cache) + off, lds);
      }
    }
    return pg_ok;
  };

  auto compute = [&](int32_t t, int slot, uint32_t pg_ok) {  // pg_ok: the tile's page validity, from its issue
    const uint8_t* K = &sm_ring[slot * SLOT];
    const int32_t k0 = TK * t;
    // a full tile: every key valid and visible to every row of the block
    const bool full = pg_ok == (1u << (TK / 16)) - 1 && k0 + TK - 1 <= pos0 &&
                      (a.window == 0 || k0 > hi - 1 - a.window);
    // S^T for each sub-tile of 32 keys (both 16-key halves) and both N tiles
    f32x4_t st[NSUB][2][2];
#pragma unroll
    for (int u = 0; u < NSUB; ++u)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int n = 0; n < 2; ++n) st[u][h][n] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < NSUB; ++u) {
      if constexpr (ESZ == 2) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          // bf16 K: elements 32 s + 8 g4 .. + 7 of the lane's key, one 16-byte LDS read per step
          const uint8_t* kr = K + (32 * u + 8 * (li >> 2) + 4 * h + (li & 3)) * RS + 16 * g4;
#pragma unroll
          for (int s = 0; s < NS; ++s) {
            const uint4 w = *reinterpret_cast<const uint4*>(kr + 64 * s);
            const uint32_t kop[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int n = 0; n < 2; ++n) st[u][h][n] = mfma_16x16x32_bf16(kop, qf[n][s], st[u][h][n]);
          }
        }
      }
      if constexpr (ESZ == 1) {
        // the K bytes of the lane's key in each half, dims 32 g4 .. + 31, straight from LDS (e4m3fn, no
        // conversion); the four (half, N tile) products' hi parts first, then their lo parts, so no MFMA waits on
        // the one before it
        uint32_t kop[2][8];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
          for (int e = 0; e < 8; ++e) kop[h][e] = 0;
          if (32 * g4 < D) {
            const uint8_t* kr = K + (32 * u + 8 * (li >> 2) + 4 * h + (li & 3)) * RS + 32 * g4;
            const uint4 w0 = *reinterpret_cast<const uint4*>(kr), w1 = *reinterpret_cast<const uint4*>(kr + 16);
            kop[h][0] = w0.x, kop[h][1] = w0.y, kop[h][2] = w0.z, kop[h][3] = w0.w;
            kop[h][4] = w1.x, kop[h][5] = w1.y, kop[h][6] = w1.z, kop[h][7] = w1.w;
          }
        }
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int n = 0; n < 2; ++n) st[u][h][n] = mfma_16x16x128_fp8(kop[h], qhi[n], st[u][h][n], qsc_hi[n]);
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int n = 0; n < 2; ++n) st[u][h][n] = mfma_16x16x128_fp8(kop[h], qlo[n], st[u][h][n], qsc_lo[n]);
      }
    }
    // scores (log2 domain) of keys k0 + 32 u + 8 g4 + j, j = 4 h + r; a tile that is not full masks them in one block
    float x[NSUB][2][8], tmax[2];
#pragma unroll
    for (int u = 0; u < NSUB; ++u)
#pragma unroll
      for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int j = 0; j < 8; ++j) x[u][n][j] = st[u][j >> 2][n][j & 3];  // raw: qk_scale (> 0) joins later
    if (!full) {
#pragma unroll
      for (int u = 0; u < NSUB; ++u) {
        // the lane's keys k0 + 32 u + 8 g4 + j all lie in 16-key group 2 u + g4 / 2
        const bool page_ok = (pg_ok >> (2 * u + (g4 >> 1))) & 1u;
        const int32_t key0 = k0 + 32 * u + 8 * g4;
#pragma unroll
        for (int n = 0; n < 2; ++n) {
          const int32_t lo_n = a.window > 0 ? qpos[n] - a.window + 1 : INT32_MIN;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int32_t key = key0 + j;
            const bool vis = page_ok & (key <= qpos[n]) & (key >= lo_n);
            x[u][n][j] = vis ? x[u][n][j] : -INFINITY;
          }
        }
      }
    }
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      float m = x[0][n][0];
#pragma unroll
      for (int u = 0; u < NSUB; ++u)
#pragma unroll
        for (int j = 0; j < 8; ++j) m = fmaxf(m, x[u][n][j]);
      tmax[n] = max_across_groups(m) * qk_scale;
    }
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      if (__any(tmax[n] > m_ref[n] + kPrefillRescaleSlack)) {
        const float m_new = tmax[n] > m_ref[n] + kPrefillRescaleSlack ? tmax[n] : m_ref[n];
        const float alpha = __builtin_amdgcn_exp2f(m_ref[n] - m_new);
        m_ref[n] = m_new;
        l_run[n] *= alpha;
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[n][c] *= alpha;
      }
    }
    if constexpr (ESZ == 2) __syncthreads();  // sm_vt holds this tile's V^T (every wave's quarter)
    const uint8_t* Vt = &sm_ring[slot * SLOT] + HALF;
    const bool vclean = pg_ok == (1u << (TK / 16)) - 1 && k0 + TK <= hi;
#pragma unroll
    for (int u = 0; u < NSUB; ++u) {
      uint32_t pop[2][4];
#pragma unroll
      for (int n = 0; n < 2; ++n) {
        float p[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) p[j] = __builtin_amdgcn_exp2f(fmaf(x[u][n][j], qk_scale, -m_ref[n]));
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          pop[n][k] = pack_bf16x2(p[2 * k], p[2 * k + 1]);
          // the row sum adds the bf16 probabilities the numerator weighs (v_dot2 with a pair of ones)
          l_run[n] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, pop[n][k]),
                                                     __builtin_bit_cast(bf16x2_t, 0x3f803f80u), l_run[n], false);
        }
      }
      const uint8_t* Vr = &sm_vt[li * Geo::VT_RS + (32 * u + 8 * g4) * 2];
      uint32_t vm0 = 0xffffffffu, vm1 = 0xffffffffu;
      if (ESZ == 1 && !vclean) {
        const bool page_ok = (pg_ok >> (2 * u + (g4 >> 1))) & 1u;
        const int32_t nvalid = page_ok ? min(max(hi - (k0 + 32 * u + 8 * g4), 0), 8) : 0;  // keys below hi
        vm0 = nvalid >= 4 ? 0xffffffffu : (1u << (8 * nvalid)) - 1u;
        vm1 = nvalid >= 8 ? 0xffffffffu : nvalid <= 4 ? 0u : (1u << (8 * (nvalid - 4))) - 1u;
      }
      uint2 vraw[NC];
      if constexpr (ESZ == 1) {
#pragma unroll
        for (int c = 0; c < NC; ++c) vraw[c] = lds_read_tr8(Vt + (32 * u + 8 * g4 + (li >> 1)) * RS + 8 * (li & 1) + 16 * c);
      }
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        uint32_t vop[4];
        if constexpr (ESZ == 1) {
          fp8x4_to_bf16x4(vraw[c].x & vm0, vop[0], vop[1]);
          fp8x4_to_bf16x4(vraw[c].y & vm1, vop[2], vop[3]);
        } else {
          const uint4 w = *reinterpret_cast<const uint4*>(Vr + 16 * c * Geo::VT_RS);
          vop[0] = w.x, vop[1] = w.y, vop[2] = w.z, vop[3] = w.w;
        }
#pragma unroll
        for (int n = 0; n < 2; ++n) acc[n][c] = mfma_16x16x32_bf16(vop, pop[n], acc[n][c]);
      }
    }
  };

  // bf16 pools (FP8 tiles read V^T straight from the ring): tile t's V (ring slot `slot`) into sm_vt as V^T. Pair
  // e = (sub-tile u, dim tile c) of the tile's NSUB x NC goes to wave e % 4, whose lane (g4, i) reads keys
  // 32 u + 8 g4 .. + 7 at dim 16 c + i and stores the 16 bytes at row 16 c + i. Keys no row may see (past the chunk
  // or on an invalid page) are zeroed, since a stale NaN would survive p = 0.
  auto convert_v = [&](int32_t t, int slot, uint32_t pg_ok) {
    constexpr int NQ = NSUB * NC / 4;  // this wave's (sub-tile, dim tile) pairs
    const uint8_t* V = &sm_ring[slot * SLOT] + HALF;
    const int32_t k0 = TK * t;
    const bool clean = pg_ok == (1u << (TK / 16)) - 1 && k0 + TK <= hi;
    // every pair's LDS reads first, then the V^T stores: a store between two reads would hold the second read back
    // until the first has returned (the compiler cannot tell the two arrays apart here)
    uint32_t raw[NQ][8];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int e = wave + 4 * q;
      const int u = e / NC, c = e % NC;
      // the 8 keys' elements at dim 16 c + i, one 2-byte LDS read each
      const uint8_t* vr = V + (32 * u + 8 * g4) * RS + 2 * (16 * c + li);
#pragma unroll
      for (int k = 0; k < 8; ++k) raw[q][k] = *reinterpret_cast<const uint16_t*>(vr + k * RS);
    }
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int e = wave + 4 * q;
      const int u = e / NC, c = e % NC;
      int32_t nvalid = 8;  // keys below hi on a valid page
      if (!clean) {
        const bool page_ok = (pg_ok >> (2 * u + (g4 >> 1))) & 1u;
        nvalid = page_ok ? min(max(hi - (k0 + 32 * u + 8 * g4), 0), 8) : 0;
      }
      uint32_t o[4];
#pragma unroll
      for (int k = 0; k < 4; ++k)
        o[k] = (2 * k < nvalid ? raw[q][2 * k] : 0u) | ((2 * k + 1 < nvalid ? raw[q][2 * k + 1] : 0u) << 16);
      *reinterpret_cast<uint4*>(&sm_vt[(16 * c + li) * Geo::VT_RS + (32 * u + 8 * g4) * 2]) = make_uint4(o[0], o[1], o[2],
                                                                                                       o[3]);
    }
  };

  // The compiler's own loads (the query operand) complete here, in a wait it sees, before any DMA is in flight.
  __builtin_amdgcn_s_waitcnt(0x0f70);

  const int32_t t_first = lo / TK, t_end = (hi + TK - 1) / TK;
  const int32_t chunk_tiles = (Geo::PAGES - 1) * a.P / TK;  // (a chunk may start mid-page: PAGES - 1 whole pages)
  for (int32_t c0 = t_first; c0 < t_end; c0 += chunk_tiles) {
    const int32_t c1 = min(c0 + chunk_tiles, t_end);
    // stage the table entries of pages [p0, p1) (ring and pages are free: the previous chunk drained)
    __syncthreads();
    p0 = TK * c0 / a.P;
    const int32_t p1 = (TK * c1 - 1) / a.P + 1;
    const int32_t* trow = a.table + (int64_t)r * a.table_stride;
    for (int32_t i = tid; i < p1 - p0; i += 256) {
      const int32_t col = p0 + i;
      const int32_t e = col < a.table_width ? trow[col] : -1;
      sm_pages[i] = (e >= 0 && (int64_t)e < a.num_blocks) ? e : -1;
    }
    __syncthreads();
    const int32_t n = c1 - c0;
    static_assert(DEPTH == 2, "tile i + 1 loads while tile i computes");
    uint32_t pg_cur = issue(c0, 0);
    for (int32_t i = 0; i < n; ++i) {
      wait_vmcnt<0>();  // this wave's DMAs of tile i have landed (tile i + 1 is not issued yet)
      // every wave's DMAs of tile i have landed; every wave is done with tile i - 1 (its slot and sm_vt are free)
      __syncthreads();
      const uint32_t pg_next = i + 1 < n ? issue(c0 + i + 1, (i + 1) % DEPTH) : 0u;
      if constexpr (ESZ == 2) convert_v(c0 + i, i % DEPTH, pg_cur);
      compute(c0 + i, i % DEPTH, pg_cur);
      pg_cur = pg_next;
    }
  }

  // ---- epilogue: normalize (sinks join the denominator), scale by v_scale, write the valid rows ----
#pragma unroll
  for (int n = 0; n < 2; ++n) {
    float L = sum_across_groups(l_run[n]);
    if (a.sinks) L += __builtin_amdgcn_exp2f(a.sinks[head[n]] * kLog2e - m_ref[n]);
    const float inv = v_scale / L;
    if (!row_ok[n]) continue;
    uint16_t* dst = a.out + ((int64_t)tok[n] * a.H + head[n]) * D + 4 * g4;
#pragma unroll
    for (int c = 0; c < NC; ++c)
      *reinterpret_cast<uint2*>(dst + 16 * c) = make_uint2(pack_bf16x2(acc[n][c][0] * inv, acc[n][c][1] * inv),
                                                           pack_bf16x2(acc[n][c][2] * inv, acc[n][c][3] * inv));
  }
}

}  // namespace sna

using namespace sna;

extern "C" int sna_prefill_attention(const void* q, const void* k_cache, const void* v_cache, const float* k_scale,
                                     const float* v_scale, const int32_t* block_table, int64_t table_stride,
                                     int32_t table_width, const int32_t* q_start, const int32_t* prior_lens,
                                     int32_t R, int32_t max_q_len, const float* sinks, float sm_scale, int32_t window,
                                     void* out, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                     int32_t page_size, int64_t num_blocks, int32_t kv_dtype, void* stream) {
  ApiGuard guard;
  if (R < 0 || max_q_len < 0 || num_q_heads < 1 || num_kv_heads < 1 || num_q_heads % num_kv_heads != 0 ||
      window < 0 || num_blocks < 1 || table_width < 1 || table_stride < table_width)
    return fail(SNA_ERR_INVALID_ARGUMENT,
                "prefill_attention: bad sizes (R %d, max_q_len %d, heads %d / %d, window %d, blocks %lld, table %d "
                "wide, stride %lld)",
                R, max_q_len, num_q_heads, num_kv_heads, window, (long long)num_blocks, table_width,
                (long long)table_stride);
  const int32_t group = num_q_heads / num_kv_heads;
  if (group > 128) return fail(SNA_ERR_UNSUPPORTED, "prefill_attention: %d query heads per KV head (at most 128)", group);
  if (head_dim != 64 && head_dim != 128)
    return fail(SNA_ERR_UNSUPPORTED, "prefill_attention: head_dim %d (64 or 128)", head_dim);
  if (page_size < 16 || page_size % 16 != 0)
    return fail(SNA_ERR_UNSUPPORTED, "prefill_attention: page_size %d (a multiple of 16)", page_size);
  if (kv_dtype != SNA_DTYPE_FP8_E4M3FN && kv_dtype != SNA_DTYPE_FP8_E4M3FN_MUL && kv_dtype != SNA_DTYPE_BF16)
    return fail(SNA_ERR_UNSUPPORTED, "prefill_attention: KV dtype %d (FP8 e4m3fn or bf16)", kv_dtype);
  if (R == 0 || max_q_len == 0) return SNA_OK;
  if (!q || !k_cache || !v_cache || (kv_dtype != SNA_DTYPE_BF16 && (!k_scale || !v_scale)) || !block_table ||
      !q_start || !prior_lens || !out)
    return fail(SNA_ERR_INVALID_ARGUMENT, "prefill_attention: null pointer");
  if (!aligned(q, 16) || !aligned(out, 16) || !aligned(k_cache, 16) || !aligned(v_cache, 16))
    return fail(SNA_ERR_INVALID_ARGUMENT, "prefill_attention: q, out and the caches must be 16-byte aligned");
  if (R > 65535 || num_kv_heads > 65535)
    return fail(SNA_ERR_INVALID_ARGUMENT, "prefill_attention: %d requests x %d KV heads exceed the grid", R,
                num_kv_heads);
  PrefillArgs a;
  a.q = (const uint16_t*)q;
  a.k_cache = (const uint8_t*)k_cache;
  a.v_cache = (const uint8_t*)v_cache;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  a.mul_scale = kv_dtype == SNA_DTYPE_FP8_E4M3FN_MUL;
  a.table = block_table;
  a.table_stride = table_stride;
  a.table_width = table_width;
  a.q_start = q_start;
  a.prior = prior_lens;
  a.sinks = sinks;
  a.out = (uint16_t*)out;
  a.R = R;
  a.H = num_q_heads;
  a.G = num_kv_heads;
  a.P = page_size;
  a.group = group;
  a.bq = 128 / group;
  a.num_blocks = num_blocks;
  a.sm_scale = sm_scale;
  a.window = window;
  const int64_t qblocks = (max_q_len + a.bq - 1) / a.bq;
  if (qblocks * R * num_kv_heads > (int64_t)UINT32_MAX)  // the kernel's XCD-aware order numbers them in 32 bits
    return fail(SNA_ERR_INVALID_ARGUMENT, "prefill_attention: %lld query blocks x %d requests x %d KV heads exceed "
                "the grid (split the batch)", (long long)qblocks, R, num_kv_heads);
  const dim3 grid((unsigned)qblocks, (unsigned)R, (unsigned)num_kv_heads);
  const int esz = kv_dtype == SNA_DTYPE_BF16 ? 2 : 1;
  const bool buf = num_blocks * num_kv_heads * (int64_t)page_size * head_dim * esz < ((int64_t)1 << 32);
  const hipStream_t s = (hipStream_t)stream;
#define SNA_PREFILL_LAUNCH(D_, BUF_, ESZ_) \
  hipLaunchKernelGGL((prefill_gqa_kernel<D_, BUF_, ESZ_>), grid, dim3(256), 0, s, a)
  if (esz == 1) {
    if (head_dim == 128) {
      if (buf) SNA_PREFILL_LAUNCH(128, true, 1); else SNA_PREFILL_LAUNCH(128, false, 1);
    } else {
      if (buf) SNA_PREFILL_LAUNCH(64, true, 1); else SNA_PREFILL_LAUNCH(64, false, 1);
    }
  } else {
    if (head_dim == 128) {
      if (buf) SNA_PREFILL_LAUNCH(128, true, 2); else SNA_PREFILL_LAUNCH(128, false, 2);
    } else {
      if (buf) SNA_PREFILL_LAUNCH(64, true, 2); else SNA_PREFILL_LAUNCH(64, false, 2);
    }
  }
#undef SNA_PREFILL_LAUNCH
  return check_launch("prefill_attention");
}
