// The DeepSeek-sparse-attention indexer's decode step on the GPU, after the model's projections: the fp8 index-key
// store, the head-weighted ReLU score of every cached key, and the exact top-k selection of the positions the sparse
// MLA decode then gathers.
//   reference: models/glm52/kernels/decode/attention/indexer/indexer_torch.py (pack_indexer_keys_fp8 :44-53, the
//   score of indexer_kv_score_torch_ref :254-268, indexer_topk_local_torch_ref :296-309)
//
// Score: one workgroup of 4 waves per (row, 2048 keys); each wave takes 16-key tiles. S[head, key] = Q . K^T on
// v_mfma_scale_f32_16x16x128_f8f6f4 (one instruction covers d = 128): lane (g4, i) feeds row i of the head tile (the
// query split exactly into two e4m3fn parts, hi + lo / 16, of a power-of-two-scaled row, whose E8M0 A scales undo
// the scaling) and column i, the 32 key bytes 32 g4 .. + 31 of key i, loaded straight from HBM into a register ring.
// The result hands lane (g4, i) heads 4 g4 + r of key i: the head-weighted ReLU sum is 16 terms in the lane, then a
// sum over the four lane groups. Bytes per key: 128 (the fp8 row) + 2 (the bf16 score written).
//
// Top-k: a two-byte radix select over order-preserving 16-bit keys of the scores, the row cut into segments of 8192
// scores, in four launches that publish per-segment histograms and counts to a workspace (described below).

#include "sna_device.h"
#include "sna_host.h"

namespace sna {

constexpr float kIndexMaskBound = 1.0e30f;

struct IndexerArgs {
  const uint16_t* q;     // [B, H, 128] bf16, rotated
  const float* w;        // [B, H] fp32 head weights (already scaled)
  const uint8_t* keys;   // [num_blocks, P, 128] e4m3fn
  const int32_t* table;  // [B, table_width] (row stride table_stride)
  int64_t table_stride;
  int32_t table_width;
  const int32_t* limits;  // [B] keys e < limits[b] are resident
  uint16_t* out;          // [B, width] bf16 (row stride out_stride)
  int64_t out_stride;
  int32_t B, H, width, P;
  int64_t num_blocks;
  float scale;  // d^-0.5
};

__device__ __forceinline__ f32x4_t mfma_16x16x128_fp8_sa(const uint32_t (&a)[8], const uint32_t (&b)[8], f32x4_t c,
                                                        int32_t scale_a) {
  i32x8_t av, bv;
#pragma unroll
  for (int i = 0; i < 8; ++i) av[i] = (int32_t)a[i], bv[i] = (int32_t)b[i];
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, c, 0, 0, 0, scale_a, 0, 127);
}

constexpr int kScoreKeys = 2048;  // keys per workgroup (a multiple of 64): 32 tiles of 16 keys per wave

template <int HT>  // head tiles of 16
__global__ __launch_bounds__(256) void indexer_score_kernel(IndexerArgs a) {
  // PD: key tiles each wave has in flight ahead of the one it scores (fewer with 128 heads, whose query operands
  // take 128 VGPRs)
  constexpr int D = 128, TILES = kScoreKeys / 64, PD = HT >= 8 ? 2 : 4;
  static_assert(kScoreKeys % 64 == 0 && kScoreKeys / 64 <= 32, "a 32-bit mask of live tiles");
  __shared__ uint32_t sm_q[HT][2][8][64];  // [head tile][hi, lo][dword][lane]: the MFMA A operand of each lane
  __shared__ int32_t sm_ex[HT][64];         // floor(log2 amax) of the head lane (li) feeds, per head tile
  __shared__ __align__(16) uint16_t sm_out[kScoreKeys];  // the workgroup's bf16 scores
  const int tid = threadIdx.x, lane = tid & 63, g4 = lane >> 4, li = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int32_t b = blockIdx.y;
  const int32_t e_blk = (int32_t)blockIdx.x * kScoreKeys;
  if (e_blk >= a.width) return;
  const int32_t limit = a.limits[b];
  const int32_t* trow = a.table + (int64_t)b * a.table_stride;

  // the raw query rows this wave splits (head tiles wave, wave + 4, ...), loaded before anything they wait on
  constexpr int QT = (HT + 3) / 4;
  uint4 qraw[QT][4];
#pragma unroll
  for (int j = 0; j < QT; ++j) {
    const int ht = wave + 4 * j;
    if (ht < HT) {
      const uint16_t* qp = a.q + ((int64_t)b * a.H + 16 * ht + li) * D + 32 * g4;
#pragma unroll
      for (int c = 0; c < 4; ++c) qraw[j][c] = ld16(qp + 8 * c);
    }
  }

  // This lane's key of tile t is e_blk + 64 t + 16 wave + li (the four waves cover 64 consecutive keys per step);
  // its page is looked up first, all tiles at once. Bit t of live_bits: the key is resident, its page valid.
  // (col, off) = divmod(e, P), stepped by 64 keys per tile: one division for the first tile, then
  // (col, off) += divmod(64, P) with at most one carry.
  int32_t kofs[TILES];  // the key row's byte offset in the cache / 16 (the cache is under 2^35 bytes), if live
  uint32_t live_bits = 0;
  {
    const int32_t e0 = e_blk + 16 * wave + li, step_col = 64 / a.P, step_off = 64 % a.P;
    int32_t col = e0 / a.P, off = e0 - col * a.P;
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
      const int32_t e = e0 + 64 * t;
      const int32_t page = (e < a.width && col < a.table_width) ? trow[col] : -1;
      const bool live = e < limit && page >= 0 && (int64_t)page < a.num_blocks;
      live_bits |= live ? (1u << t) : 0u;
      kofs[t] = live ? (int32_t)((((int64_t)page * a.P + off) * D) >> 4) : 0;
      col += step_col;
      off += step_off;
      if (off >= a.P) off -= a.P, ++col;
    }
  }

  // key tiles in flight: tile t's 32 bytes of this lane land in ring[t % PD]. Every lane loads (a dead key reads
  // row 0 of the cache, in bounds, and its score is replaced), so no branch or store sits between a load and its
  // use and the waits count only the ring's own loads.
  uint32_t ring[PD][8];
  auto fetch = [&](int t, uint32_t (&kb)[8]) {
    const uint8_t* kp = a.keys + ((int64_t)kofs[t] << 4) + 32 * g4;
    // plain loads: with the non-temporal hint the same stream measured ~3% slower
    const uint4 x0 = ld16(kp), x1 = ld16(kp + 16);
    kb[0] = x0.x, kb[1] = x0.y, kb[2] = x0.z, kb[3] = x0.w, kb[4] = x1.x, kb[5] = x1.y, kb[6] = x1.z, kb[7] = x1.w;
  };
#pragma unroll
  for (int u = 0; u < PD; ++u) fetch(u, ring[u]);

  // The query operand of head tile ht: lane (g4, i) supplies head 16 ht + i, dims 32 g4 .. + 31, as two exact
  // e4m3fn parts of the row scaled by sc = 2^(7 - floor(log2 amax)) (amax over the head's 128 dims); the E8M0 A
  // scales are 127 - log2 sc for hi and 4 less for lo. Wave w splits head tiles w, w + 4, ... into LDS.
#pragma unroll
  for (int j = 0; j < QT; ++j) {
    const int ht = wave + 4 * j;
    if (ht >= HT) break;  // (uniform)
    float v[32];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint4 x = qraw[j][c];
      const uint32_t xx[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[8 * c + 2 * e] = bf16_bits_to_f32(xx[e] & 0xffffu);
        v[8 * c + 2 * e + 1] = bf16_bits_to_f32(xx[e] >> 16);
      }
    }
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 32; ++e) amax = fmaxf(amax, fabsf(v[e]));
    amax = max_across_groups(amax);
    const int32_t ex = amax > 0.0f ? max((int32_t)((__float_as_uint(amax) >> 23) & 0xff) - 127, -116) : -7;
    const float sc = __uint_as_float((uint32_t)(127 + 7 - ex) << 23);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      float h4[4], l4[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) split_q(v[4 * k + e] * sc, h4[e], l4[e]);
      sm_q[ht][0][k][lane] = pack_e4m3fn_x4(h4[0], h4[1], h4[2], h4[3]);
      sm_q[ht][1][k][lane] = pack_e4m3fn_x4(l4[0], l4[1], l4[2], l4[3]);
    }
    sm_ex[ht][lane] = ex;
  }
  // weights of heads 16 ht + 4 g4 + r (the rows this lane's results hold), times d^-0.5: w relu(s d^-0.5) =
  // (w d^-0.5) relu(s) as d^-0.5 > 0
  float wl[HT][4];
#pragma unroll
  for (int ht = 0; ht < HT; ++ht)
#pragma unroll
    for (int r = 0; r < 4; ++r) wl[ht][r] = a.w[(int64_t)b * a.H + 16 * ht + 4 * g4 + r] * a.scale;

  __syncthreads();
  uint32_t qhi[HT][8], qlo[HT][8];
  int32_t sc_hi[HT], sc_lo[HT];
#pragma unroll
  for (int ht = 0; ht < HT; ++ht) {
#pragma unroll
    for (int k = 0; k < 8; ++k) qhi[ht][k] = sm_q[ht][0][k][lane], qlo[ht][k] = sm_q[ht][1][k][lane];
    const int32_t ex = sm_ex[ht][lane];
    sc_hi[ht] = 127 + ex - 7;
    sc_lo[ht] = 127 + ex - 7 - 4;
  }

  // scores of the workgroup's keys, written out coalesced at the end
#pragma unroll
  for (int t = 0; t < TILES; ++t) {
    float sum = 0.0f;
#pragma unroll
    for (int ht = 0; ht < HT; ++ht) {
      f32x4_t s = {0.f, 0.f, 0.f, 0.f};
      s = mfma_16x16x128_fp8_sa(qhi[ht], ring[t % PD], s, sc_hi[ht]);
      s = mfma_16x16x128_fp8_sa(qlo[ht], ring[t % PD], s, sc_lo[ht]);
#pragma unroll
      for (int r = 0; r < 4; ++r)  // relu as an integer max: a negative float's bits are a negative integer
        sum = fmaf(wl[ht][r], __int_as_float(max(__float_as_int(s[r]), 0)), sum);
    }
    if (t + PD < TILES) fetch(t + PD, ring[t % PD]);
    sum = sum_across_groups(sum);  // every lane of key li holds the key's sum
    const bool live = (live_bits >> t) & 1u;
    sm_out[64 * t + 16 * wave + li] = (uint16_t)f32_to_bf16_bits(live ? fminf(sum, kIndexMaskBound) : -kIndexMaskBound);
  }
  __syncthreads();
  uint16_t* orow = a.out + (int64_t)b * a.out_stride + e_blk;
  const int32_t n = min(kScoreKeys, a.width - e_blk);
  if (n == kScoreKeys && ((uintptr_t)orow & 7) == 0) {
    for (int32_t i = 4 * tid; i < kScoreKeys; i += 4 * 256)
      *reinterpret_cast<uint2*>(orow + i) = *reinterpret_cast<const uint2*>(&sm_out[i]);
  } else {
    for (int32_t i = tid; i < n; i += 256) orow[i] = sm_out[i];
  }
}

// bf16 bits -> a 16-bit key whose unsigned order is the value order (NaN aside).
__device__ __forceinline__ uint32_t order_key(uint32_t bits) { return (bits & 0x8000u) ? (~bits & 0xffffu) : (bits | 0x8000u); }
__device__ __forceinline__ uint32_t key_bits(uint32_t key) { return (key & 0x8000u) ? (key & 0x7fffu) : (~key & 0xffffu); }

// ---- top-k: a two-byte radix select over the rows' segments ----
// A row of bf16 scores is cut into segments of kTopkSeg scores, one workgroup of 1024 lanes (8 scores each, one
// 16-byte load) per (segment, row). Scores compare through order_key, a 16-bit key that sorts as the value does. Four
// launches, each workgroup reading only what earlier launches published in the workspace (no zeroing, no global
// atomics):
//   topk_hist_hi:  the segment's histogram of the key's high byte          -> hist_hi[b][s][256]
//   topk_hist_lo:  the row's bin H holding the k-th largest key (summing hist_hi over the segments);
//                  the segment's histogram of the low byte of keys in H    -> hist_lo[b][s][256]
//   topk_count:    the threshold key T (the k-th largest) and the count above it; the segment's counts of keys
//                  above and equal to T                                    -> counts[b][s], and sel[b] from s = 0
//   topk_write:    positions in order: keys above T at the running count of those before them, then T's ties at
//                  n_above + their running count, while that is below k.
// Workspace per row: (2 * 256 + 1) * S + 4 u32, S = ceil(width / kTopkSeg).
constexpr int kTopkSeg = 8192, kTopkCopies = 32;

struct TopkRow {
  const uint16_t* row;  // this row's scores
  uint32_t* hist_hi;    // [S][256]
  uint32_t* hist_lo;    // [S][256]
  uint32_t* counts;     // [S]: (ties << 16) | above
  uint32_t* sel;        // [4]: T, n_above
};

__device__ __forceinline__ TopkRow topk_row(const uint16_t* scores, int64_t score_stride, uint32_t* ws, int32_t S) {
  const int32_t b = blockIdx.y;
  uint32_t* base = ws + (int64_t)b * ((2 * 256 + 1) * (int64_t)S + 4);
  return {scores + (int64_t)b * score_stride, base, base + 256 * S, base + 512 * S, base + 513 * S};
}

// this lane's 8 keys of segment blockIdx.x (past the row: key 0, never counted); in[j] says whether key j is inside
__device__ __forceinline__ void topk_keys(const uint16_t* row, bool vec, int32_t width, uint32_t (&key)[8]) {
  const int32_t e = blockIdx.x * kTopkSeg + 8 * threadIdx.x;
  if (vec && e + 8 <= width) {
    const uint4 v = *reinterpret_cast<const uint4*>(row + e);
    const uint32_t x[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) key[j] = order_key((x[j >> 1] >> (16 * (j & 1))) & 0xffffu);
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) key[j] = e + j < width ? order_key(row[e + j]) : 0u;
  }
}

__device__ __forceinline__ bool topk_vec(const uint16_t* scores, int64_t score_stride) {
  return (score_stride % 8) == 0 && ((uintptr_t)scores & 15) == 0;  // rows 16-byte aligned: 8 scores per load
}

// LDS histogram helpers: 256 bins x kTopkCopies copies, bin-major; lane l adds into copy l mod 32, so the lanes of
// one atomic instruction never share a bank
__device__ __forceinline__ void topk_clear(uint32_t* hist) {
  for (int i = threadIdx.x; i < 256 * kTopkCopies; i += blockDim.x) hist[i] = 0;
}
__device__ __forceinline__ void topk_publish(const uint32_t* hist, uint32_t* dst) {
  const int t = threadIdx.x;
  if (t < 256) {
    uint32_t c = 0;
#pragma unroll 8
    for (int i = 0; i < kTopkCopies; ++i) c += hist[t * kTopkCopies + ((i + t) & (kTopkCopies - 1))];
    dst[t] = c;
  }
}

// The bin (from the top) where the running count of the row's keys, over the S published histograms hist[S][256],
// reaches `need`, and the count in the bins above it plus base_above; every lane gets both. Threads 0..255 take
// bin 255 - t. wtot: 4 u32 of LDS, out: 2 u32 of LDS.
__device__ __forceinline__ void topk_pick(const uint32_t* hist, int32_t S, uint32_t need, uint32_t base_above,
                                          uint32_t* wtot, uint32_t* out, uint32_t& bin, uint32_t& above) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  uint32_t cnt = 0, incl = 0;
  if (t < 256) {
    // S published histograms, written by other workgroups (other XCDs): 16 independent loads in flight at a time
    for (int32_t s0 = 0; s0 < S; s0 += 16) {
      uint32_t v[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) v[j] = s0 + j < S ? hist[(int64_t)(s0 + j) * 256 + 255 - t] : 0u;
#pragma unroll
      for (int j = 0; j < 16; ++j) cnt += v[j];
    }
    incl = cnt;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const uint32_t v = __shfl_up(incl, off, 64);
      if (lane >= off) incl += v;
    }
    if (lane == 63) wtot[wave] = incl;
  }
  __syncthreads();
  if (t < 256) {
    for (int w = 0; w < wave; ++w) incl += wtot[w];
    incl += base_above;
    const uint32_t before = incl - cnt;
    // the first bin from the top whose running count reaches need (bin 0 takes whatever is left)
    if ((before < need && incl >= need) || (t == 255 && before < need)) {
      out[0] = 255u - (uint32_t)t;
      out[1] = before;
    }
  }
  __syncthreads();
  bin = out[0];
  above = out[1];
}

__global__ __launch_bounds__(1024) void topk_hist_hi_kernel(const uint16_t* __restrict__ scores,
                                                            int64_t score_stride, int32_t width, int32_t S,
                                                            uint32_t* __restrict__ ws) {
  __shared__ uint32_t hist[256 * kTopkCopies];
  const TopkRow r = topk_row(scores, score_stride, ws, S);
  uint32_t key[8];
  topk_keys(r.row, topk_vec(scores, score_stride), width, key);
  topk_clear(hist);
  __syncthreads();
  uint32_t* mine = hist + (threadIdx.x & (kTopkCopies - 1));
  const int32_t e = blockIdx.x * kTopkSeg + 8 * threadIdx.x;
#pragma unroll
  for (int j = 0; j < 8; ++j)
    if (e + j < width) atomicAdd(&mine[(key[j] >> 8) * kTopkCopies], 1u);
  __syncthreads();
  topk_publish(hist, r.hist_hi + (int64_t)blockIdx.x * 256);
}

__global__ __launch_bounds__(1024) void topk_hist_lo_kernel(const uint16_t* __restrict__ scores,
                                                            int64_t score_stride, int32_t width, int32_t S, int32_t k,
                                                            uint32_t* __restrict__ ws) {
  __shared__ uint32_t hist[256 * kTopkCopies];
  __shared__ uint32_t wtot[4], pick[2];
  const TopkRow r = topk_row(scores, score_stride, ws, S);
  uint32_t key[8];
  topk_keys(r.row, topk_vec(scores, score_stride), width, key);
  topk_clear(hist);
  uint32_t hi, above;
  topk_pick(r.hist_hi, S, (uint32_t)k, 0, wtot, pick, hi, above);  // its barriers also cover the clear
  uint32_t* mine = hist + (threadIdx.x & (kTopkCopies - 1));
  const int32_t e = blockIdx.x * kTopkSeg + 8 * threadIdx.x;
#pragma unroll
  for (int j = 0; j < 8; ++j)
    if (e + j < width && (key[j] >> 8) == hi) atomicAdd(&mine[(key[j] & 0xffu) * kTopkCopies], 1u);
  __syncthreads();
  topk_publish(hist, r.hist_lo + (int64_t)blockIdx.x * 256);
}

// the threshold key T and the count above it, from the two published histograms
__device__ __forceinline__ void topk_threshold(const TopkRow& r, int32_t S, int32_t k, uint32_t* wtot, uint32_t* pick,
                                               uint32_t& T, uint32_t& n_above) {
  uint32_t hi, above1, lo;
  topk_pick(r.hist_hi, S, (uint32_t)k, 0, wtot, pick, hi, above1);
  __syncthreads();  // pick[] is rewritten
  topk_pick(r.hist_lo, S, (uint32_t)k, above1, wtot, pick, lo, n_above);
  T = (hi << 8) | lo;
}

__global__ __launch_bounds__(1024) void topk_count_kernel(const uint16_t* __restrict__ scores, int64_t score_stride,
                                                          int32_t width, int32_t S, int32_t k,
                                                          uint32_t* __restrict__ ws) {
  __shared__ uint32_t wtot[16], pick[2];
  const TopkRow r = topk_row(scores, score_stride, ws, S);
  uint32_t key[8];
  topk_keys(r.row, topk_vec(scores, score_stride), width, key);
  uint32_t T, n_above;
  topk_threshold(r, S, k, wtot, pick, T, n_above);
  const int32_t e = blockIdx.x * kTopkSeg + 8 * threadIdx.x;
  uint32_t cnt = 0;  // (ties << 16) | above, each at most 8 per lane and kTopkSeg per segment
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const bool in = e + j < width;
    cnt += (in && key[j] > T) ? 1u : 0u;
    cnt += (in && key[j] == T) ? 0x10000u : 0u;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) cnt += __shfl_xor(cnt, off, 64);
  __syncthreads();  // wtot was read by the picks
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) wtot[wave] = cnt;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t total = 0;
    for (int w = 0; w < 16; ++w) total += wtot[w];
    r.counts[blockIdx.x] = total;
    if (blockIdx.x == 0) {
      r.sel[0] = T;
      r.sel[1] = n_above;
    }
  }
}

__global__ __launch_bounds__(1024) void topk_write_kernel(const uint16_t* __restrict__ scores, int64_t score_stride,
                                                          int32_t width, int32_t S, int32_t k,
                                                          uint32_t* __restrict__ ws, int32_t* __restrict__ out,
                                                          int64_t out_stride) {
  __shared__ uint32_t wtot[16];
  const TopkRow r = topk_row(scores, score_stride, ws, S);
  uint32_t key[8];
  topk_keys(r.row, topk_vec(scores, score_stride), width, key);
  const uint32_t T = r.sel[0], n_above = r.sel[1], n_ties = (uint32_t)k - n_above;
  uint32_t run_gt = 0, run_eq = 0;  // the counts of the segments before this one (ties may pass 16 bits here)
  for (int32_t s0 = 0; s0 < (int32_t)blockIdx.x; s0 += 16) {
    uint32_t c[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) c[j] = s0 + j < (int32_t)blockIdx.x ? r.counts[s0 + j] : 0u;
#pragma unroll
    for (int j = 0; j < 16; ++j) run_gt += c[j] & 0xffffu, run_eq += c[j] >> 16;
  }
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int32_t e = blockIdx.x * kTopkSeg + 8 * tid;
  uint32_t cnt = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const bool in = e + j < width;
    cnt += (in && key[j] > T) ? 1u : 0u;
    cnt += (in && key[j] == T) ? 0x10000u : 0u;
  }
  uint32_t incl = cnt;  // inclusive scan over the wave
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t v = __shfl_up(incl, off, 64);
    if (lane >= off) incl += v;
  }
  if (lane == 63) wtot[wave] = incl;
  __syncthreads();
  uint32_t before = 0;  // packed: inside one segment each count is at most kTopkSeg
#pragma unroll
  for (int w = 0; w < 16; ++w) before += w < wave ? wtot[w] : 0u;
  const uint32_t excl = before + incl - cnt;
  uint32_t o_gt = run_gt + (excl & 0xffffu), o_eq = run_eq + (excl >> 16);
  int32_t* orow = out + (int64_t)blockIdx.y * out_stride;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if (e + j >= width) continue;
    const int32_t label = bf16_bits_to_f32(key_bits(key[j])) > -0.5f * kIndexMaskBound ? e + j : -1;  // dead: -1
    if (key[j] > T) {
      orow[o_gt++] = label;
    } else if (key[j] == T) {
      if (o_eq < n_ties) orow[n_above + o_eq] = label;
      ++o_eq;
    }
  }
}

// e4m3fn(clamp(key, +-448)) rows into an index-key cache; one thread per 8 elements, out-of-cache slots skipped.
__global__ __launch_bounds__(256) void index_key_store_kernel(const uint16_t* __restrict__ keys, const int64_t* slots,
                                                              int64_t n, int32_t d, uint8_t* cache, int64_t n_slots) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int32_t per_row = d / 8;
  if (i >= n * per_row) return;
  const int64_t t = i / per_row;
  const int32_t c = (int32_t)(i % per_row);
  const int64_t s = slots[t];
  if (s < 0 || s >= n_slots) return;
  const uint4 x = ld16(keys + t * d + 8 * c);
  const uint32_t xx[4] = {x.x, x.y, x.z, x.w};
  uint32_t o[2] = {0, 0};
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j >> 2] |= quantize_e4m3fn((xx[j >> 1] >> (16 * (j & 1))) & 0xffffu, 1.0f) << (8 * (j & 3));
  *reinterpret_cast<uint2*>(cache + s * d + 8 * c) = make_uint2(o[0], o[1]);
}

}  // namespace sna

using namespace sna;

extern "C" {

int sna_indexer_scores(const void* q, const float* w, const uint8_t* keys, const int32_t* block_table,
                       int64_t table_stride, int32_t table_width, const int32_t* limits, int32_t B, int32_t num_heads,
                       int32_t head_dim, int32_t page_size, int64_t num_blocks, int32_t width, void* out,
                       int64_t out_stride, void* stream) {
  ApiGuard guard;
  if (B < 0 || width < 0 || num_heads < 16 || num_heads % 16 != 0 || num_heads > 128 || page_size < 1 ||
      num_blocks < 1 || table_width < 1 || table_stride < table_width || out_stride < width)
    return fail(SNA_ERR_INVALID_ARGUMENT,
                "indexer_scores: bad sizes (B %d, heads %d (a multiple of 16, at most 128), page %d, blocks %lld, "
                "table %d wide, width %d, out stride %lld)",
                B, num_heads, page_size, (long long)num_blocks, table_width, width, (long long)out_stride);
  if (head_dim != 128) return fail(SNA_ERR_UNSUPPORTED, "indexer_scores: head_dim %d (128)", head_dim);
  if (B == 0 || width == 0) return SNA_OK;
  if (!q || !w || !keys || !block_table || !limits || !out)
    return fail(SNA_ERR_INVALID_ARGUMENT, "indexer_scores: null pointer");
  if (!aligned(q, 16) || !aligned(keys, 16)) return fail(SNA_ERR_INVALID_ARGUMENT, "indexer_scores: q and keys 16-B aligned");
  if (B > 65535) return fail(SNA_ERR_INVALID_ARGUMENT, "indexer_scores: %d rows exceed the grid", B);
  if (num_blocks * (int64_t)page_size * head_dim >= ((int64_t)1 << 35))
    return fail(SNA_ERR_UNSUPPORTED, "indexer_scores: a key cache of 32 GiB or more");
  IndexerArgs a;
  a.q = (const uint16_t*)q;
  a.w = w;
  a.keys = keys;
  a.table = block_table;
  a.table_stride = table_stride;
  a.table_width = table_width;
  a.limits = limits;
  a.out = (uint16_t*)out;
  a.out_stride = out_stride;
  a.B = B;
  a.H = num_heads;
  a.width = width;
  a.P = page_size;
  a.num_blocks = num_blocks;
  a.scale = 1.0f / sqrtf((float)head_dim);
  const dim3 grid((unsigned)((width + kScoreKeys - 1) / kScoreKeys), (unsigned)B);
  const hipStream_t s = (hipStream_t)stream;
  switch (num_heads / 16) {
    case 1: hipLaunchKernelGGL((indexer_score_kernel<1>), grid, dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL((indexer_score_kernel<2>), grid, dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL((indexer_score_kernel<4>), grid, dim3(256), 0, s, a); break;
    case 8: hipLaunchKernelGGL((indexer_score_kernel<8>), grid, dim3(256), 0, s, a); break;
    default:
      return fail(SNA_ERR_UNSUPPORTED, "indexer_scores: %d heads (16, 32, 64 or 128)", num_heads);
  }
  return check_launch("indexer_scores");
}

int64_t sna_topk_workspace_bytes(int32_t B, int32_t width) {
  if (B <= 0 || width <= 0) return 0;
  const int64_t S = ((int64_t)width + kTopkSeg - 1) / kTopkSeg;
  return (int64_t)B * ((2 * 256 + 1) * S + 4) * (int64_t)sizeof(uint32_t);
}

int sna_topk_positions(const void* scores, int64_t score_stride, int32_t B, int32_t width, int32_t k, int32_t* out,
                       int64_t out_stride, void* workspace, int64_t workspace_bytes, void* stream) {
  ApiGuard guard;
  if (B < 0 || width < 0 || k < 1 || k > width || score_stride < width || out_stride < k || B > 65535)
    return fail(SNA_ERR_INVALID_ARGUMENT, "topk_positions: bad sizes (B %d, width %d, k %d, strides %lld / %lld)", B,
                width, k, (long long)score_stride, (long long)out_stride);
  if (B == 0) return SNA_OK;
  if (!scores || !out || !workspace) return fail(SNA_ERR_INVALID_ARGUMENT, "topk_positions: null pointer");
  const int64_t need = sna_topk_workspace_bytes(B, width);
  if (workspace_bytes < need)
    return fail(SNA_ERR_WORKSPACE, "topk_positions: workspace of %lld bytes, need %lld", (long long)workspace_bytes,
                (long long)need);
  if (((uintptr_t)workspace & 3) != 0) return fail(SNA_ERR_INVALID_ARGUMENT, "topk_positions: unaligned workspace");
  const int32_t S = (int32_t)(((int64_t)width + kTopkSeg - 1) / kTopkSeg);
  const dim3 grid((unsigned)S, (unsigned)B), block(1024);
  const uint16_t* sc = (const uint16_t*)scores;
  uint32_t* ws = (uint32_t*)workspace;
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(topk_hist_hi_kernel, grid, block, 0, st, sc, score_stride, width, S, ws);
  hipLaunchKernelGGL(topk_hist_lo_kernel, grid, block, 0, st, sc, score_stride, width, S, k,
                        ws);
  hipLaunchKernelGGL(topk_count_kernel, grid, block, 0, st, sc, score_stride, width, S, k, ws);
  hipLaunchKernelGGL(topk_write_kernel, grid, block, 0, st, sc, score_stride, width, S, k, ws, out,
                        out_stride);
  return check_launch("topk_positions");
}

int sna_index_key_store(const void* keys, const int64_t* slots, int64_t n_tokens, int32_t head_dim, uint8_t* cache,
                        int64_t n_slots, void* stream) {
  ApiGuard guard;
  if (n_tokens < 0 || head_dim < 8 || head_dim % 8 != 0 || n_slots < 0)
    return fail(SNA_ERR_INVALID_ARGUMENT, "index_key_store: bad sizes (tokens %lld, head_dim %d, slots %lld)",
                (long long)n_tokens, head_dim, (long long)n_slots);
  if (n_tokens == 0) return SNA_OK;
  if (!keys || !slots || !cache) return fail(SNA_ERR_INVALID_ARGUMENT, "index_key_store: null pointer");
  if (!aligned(keys, 16) || !aligned(cache, 8))
    return fail(SNA_ERR_INVALID_ARGUMENT, "index_key_store: keys 16-B and cache 8-B aligned");
  const int64_t n = n_tokens * (head_dim / 8);
  hipLaunchKernelGGL(index_key_store_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)keys, slots, n_tokens, head_dim, cache, n_slots);
  return check_launch("index_key_store");
}

}  // extern "C"
