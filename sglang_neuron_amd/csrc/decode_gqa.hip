// GQA paged decode: split-K online softmax over the block table with MFMA for QK^T and PV. The workgroup of a
// row's last split also attends the step's own token in-band and stores it into the pool. A row with one split
// writes its final output; otherwise a combine pass merges the splits and adds the sink.
//
// Work: one workgroup of 4 waves per (sequence, split, KV head). A wave takes 32-key tiles round-robin, loading the
// next tile while it computes the current one. A tile is two half-tiles of 16 keys, each inside one page (page_size
// is a multiple of 16).
//
// Lane roles in a wave (lane = 16 * g4 + li):
//   QK   S^T[key, head] = K[key, :] . Q[head, :]   with v_mfma_f32_16x16x32_bf16, M = 16 keys, N = 16 heads (the
//        group's heads, zero-padded), K = head_dim in steps of 32. Lane (g4, li) feeds key li's 16-byte chunks
//        4 c + g4 (so one load instruction reads 64 contiguous bytes of each of 16 keys) and head li's query
//        elements of the same dims. A and B use one K-index map, so the contraction pairs them however the
//        instruction orders K internally.
//   out  lane (g4, j) holds S^T[4 g4 + r, j], r = 0..3, for each half-tile: 8 keys of head j.
//   PV   O^T[d, head] = V^T[d, keys] . P^T[keys, head]   with v_mfma_f32_16x16x32_bf16, K = the tile's 32 keys,
//        ordered so that lane (g4, *) supplies keys {4 g4 .. 4 g4 + 3} of both half-tiles: exactly the probabilities
//        that lane already holds. So P never moves between lanes, and only V is transposed: lane (g4, li) loads
//        D/16 contiguous elements V[key, D/16 * li ...] of its 8 keys and regroups them in registers so that the
//        d-tile t operand holds V[8 keys, D/16 * li + t].
//   acc  lane (g4, j), d-tile t, row r accumulates O[head j, D/16 * (4 g4 + r) + t].
//
// Softmax state per head is (m, l, acc) in the log2 domain. m moves only when a tile's maximum passes it by more than
// 8 (a factor of 256), so the accumulators are rescaled rarely. Probabilities stay <= 256, which bf16 and fp32
// hold without loss of relative precision.
#include <mutex>

#include "sna_device.h"
#include "sna_host.h"

namespace sna {

constexpr float kRescaleSlack = 8.0f;

struct GqaArgs {
  const uint16_t* q;
  uint8_t* k_cache;
  uint8_t* v_cache;
  const float* k_scale;  // FP8: dequantization scales s, or (mul_scale) the GPT-OSS quantization multipliers m
  const float* v_scale;
  bool mul_scale;        // SNA_DTYPE_FP8_E4M3FN_MUL: a cached byte is worth byte / m; the own token stores bf16(x m)
  const int32_t* table;
  int64_t table_stride;
  int32_t table_width;
  const int32_t* seq_lens;
  const uint16_t* k_new;
  const uint16_t* v_new;
  const int64_t* new_slots;
  const float* sinks;
  int32_t B, H, G, group, P;
  int64_t num_blocks;
  int32_t window;
  float sm_scale;
  int32_t split_tiles;  // a device-split launch sizes its splits from the device's seq_lens (gqa_device_item)
  int32_t n_work;
  int32_t max_splits;
  int32_t dev_split;    // 1: a plan from a bound whose split size the launch computes (n_work: the items it may run)
  int32_t work_n;                       // entries of work (0: locate items from seq_lens)
  uint32_t work[SNA_MAX_WORK_MAP];      // item -> row << 6 | split (| kWorkLastSplit on a row's last), from the plan
  uint8_t row_splits[SNA_MAX_WORK_MAP]; // with a map (B <= SNA_MAX_WORK_MAP): the map's items per row
  float* ws_o;   // [B, max_splits, H, D]  unnormalized partials (V dequantized)
  float* ws_ml;  // [B, max_splits, H, 2]  reference max (log2 domain) and softmax sum
  int32_t* ws_st;  // a device split's split size, written by the decode launch for its combine (after ws_ml)
  uint16_t* out;
};

// The splits this launch runs for row b: its entries in the plan's item map (counted on the host), or (no map: items
// located from seq_lens) the device length's split count, with split size st, up to the plan's.
// A device split gives every row at least one split: a row with no prior key attends and stores its own token in a
// split of no tile (so no lone-token pass is needed).
__device__ __forceinline__ int32_t launched_splits(const GqaArgs& a, int32_t b, int32_t seq_len, int32_t st) {
  if (a.work_n > 0) return a.row_splits[b];
  const int32_t n = splits_of<32>(seq_len, a.window, st);
  return min(a.dev_split ? max(n, 1) : n, max(a.max_splits, 1));
}

template <int CTRL>
__device__ __forceinline__ int32_t dpp_i32(int32_t v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
// Inclusive prefix sum of v over the wave's 64 lanes (lane l gets v[0] + ... + v[l]), and the wave's sum in *total
// (uniform). Within each 16-lane row by row_shr 1, 2, 4 and 8 (a lane whose source lies before its row's start adds
// 0: the move leaves it the old value, 0), then each row adds the sums of the rows before it, read from their last
// lanes. VALU moves and lane reads, no LDS round trip.
__device__ __forceinline__ int32_t wave_incl_scan_i32(int32_t v, int32_t* total) {
  v += dpp_i32<0x111>(v);
  v += dpp_i32<0x112>(v);
  v += dpp_i32<0x114>(v);
  v += dpp_i32<0x118>(v);
  const int32_t r0 = __builtin_amdgcn_readlane(v, 15), r1 = __builtin_amdgcn_readlane(v, 31);
  const int32_t r2 = __builtin_amdgcn_readlane(v, 47), r3 = __builtin_amdgcn_readlane(v, 63);
  const int row = (threadIdx.x & 63) >> 4;
  *total = r0 + r1 + r2 + r3;
  return v + (row > 0 ? r0 : 0) + (row > 1 ? r1 : 0) + (row > 2 ? r2 : 0);
}
// The wave's largest v (uniform) for v >= 0: running maxima within each row the same way, then the rows' last lanes.
__device__ __forceinline__ int32_t wave_max_nonneg_i32(int32_t v) {
  v = max(v, dpp_i32<0x111>(v));
  v = max(v, dpp_i32<0x112>(v));
  v = max(v, dpp_i32<0x114>(v));
  v = max(v, dpp_i32<0x118>(v));
  return max(max(__builtin_amdgcn_readlane(v, 15), __builtin_amdgcn_readlane(v, 31)),
             max(__builtin_amdgcn_readlane(v, 47), __builtin_amdgcn_readlane(v, 63)));
}

// A device split's item (every lane of the calling wave gets the same values): the launch's split size st and, for
// item w, its row b (-1 past the last item), split and the row's seq_len L, from one load of every row's length.
// Every row has at least one split (launched_splits). The split size is the host planner's one-round rule applied
// to the device's lengths: at least 4 tiles and ceil(total tiles / items), at least min(longest row, 8) tiles, at
// most the longest row, grown to the least size whose items (sum over rows of max(1, ceil(tiles / size))) fit the
// launch's n_work, and at least a 64th of the longest row (a row's splits fit the combine's 64 weights). The least
// size is bisected between that start and ceil(total / (items - B)), which fits (each row's count is below
// tiles / size + 1). The rows' lengths and tile counts stay in registers: B <= kGqaDevSplitRows, n_work >= B (so the
// longest row's size fits) and a row spans at most kGqaDevSplitMaxTiles tiles (the planner's bound). Items are
// numbered row by row, splits in order, as locate_work numbers them.
__device__ void gqa_device_item(const GqaArgs& a, int32_t w, int32_t& b_out, int32_t& split_out, int32_t& st_out,
                                int32_t& len_out) {
  constexpr int R = kGqaDevSplitRows / 64;
  const int lane = threadIdx.x & 63;
  const int chunks = (a.B + 63) / 64;
  int32_t lens[R];
#pragma unroll
  for (int i = 0; i < R; ++i)
    if (i < chunks) lens[i] = ld_const(a.seq_lens + min(lane + 64 * i, a.B - 1));  // uniform branch: all in flight
  uint32_t tiles[R];
  int32_t lane_total = 0, lane_max = 0;
#pragma unroll
  for (int i = 0; i < R; ++i) {
    tiles[i] = 0;
    if (i < chunks && lane + 64 * i < a.B)
      tiles[i] = (uint32_t)min(splits_of<32>(lens[i], a.window, 1), kGqaDevSplitMaxTiles);
    lane_total += (int32_t)tiles[i];
    lane_max = max(lane_max, (int32_t)tiles[i]);
  }
  int32_t total;
  wave_incl_scan_i32(lane_total, &total);
  const int32_t mx = wave_max_nonneg_i32(lane_max);
  const int32_t items = max(a.n_work, a.B);
  const int32_t cap = max(mx, 4);
  int32_t lo = min(max(max(4, (total + items - 1) / items), min(mx, 8)), cap);
  int32_t hi = items > a.B ? min(cap, max(lo, (total + items - a.B - 1) / (items - a.B))) : cap;
  while (lo < hi) {  // uniform
    const uint32_t mid = (uint32_t)((lo + hi) >> 1);
    const float rmid = 1.0f / (float)mid;
    int32_t lane_n = 0;
#pragma unroll
    for (int i = 0; i < R; ++i)
      if (i < chunks && lane + 64 * i < a.B) lane_n += (int32_t)max(ceil_div_small(tiles[i], mid, rmid), 1u);
    int32_t n;
    wave_incl_scan_i32(lane_n, &n);
    if (n <= items) hi = (int32_t)mid;
    else lo = (int32_t)mid + 1;
  }
  const uint32_t st = (uint32_t)__builtin_amdgcn_readfirstlane(max(lo, (mx + kMaxSplits - 1) / kMaxSplits));
  const float rst = 1.0f / (float)st;
  st_out = (int32_t)st;
  b_out = -1;
  split_out = 0;
  len_out = 0;
  int32_t base = 0;
#pragma unroll
  for (int i = 0; i < R; ++i) {
    if (i < chunks && b_out < 0) {  // uniform
      const int32_t n = lane + 64 * i < a.B ? (int32_t)max(ceil_div_small(tiles[i], st, rst), 1u) : 0;
      int32_t part;
      const int32_t incl = wave_incl_scan_i32(n, &part);
      if (w < base + part) {
        const int32_t excl = incl - n;
        const uint64_t mine = __ballot(w >= base + excl && w < base + incl);
        const int32_t src = (int32_t)__builtin_amdgcn_readfirstlane(__ffsll((long long)mine) - 1);
        b_out = 64 * i + src;
        split_out = w - base - __builtin_amdgcn_readlane(excl, src);
        len_out = __builtin_amdgcn_readlane(lens[i], src);
      }
      base += part;
    }
  }
}

template <int NB>
__device__ __forceinline__ void load_bytes(const uint8_t* p, uint32_t (&dst)[NB / 4]) {
  static_assert(NB % 4 == 0, "whole dwords");
  if constexpr (NB % 16 == 0) {
#pragma unroll
    for (int i = 0; i < NB / 16; ++i) {
      const uint4 w = ld16_stream(p + 16 * i);
      dst[4 * i] = w.x;
      dst[4 * i + 1] = w.y;
      dst[4 * i + 2] = w.z;
      dst[4 * i + 3] = w.w;
    }
  } else if constexpr (NB == 8) {
    const uint2 w = ld8_stream(p);
    dst[0] = w.x;
    dst[1] = w.y;
  } else {
    static_assert(NB == 4, "4, 8 or a multiple of 16 bytes");
    dst[0] = ld4_stream(p);
  }
}

template <int D, bool FP8>
struct GqaTile {
  static constexpr int ESZ = FP8 ? 1 : 2;
  static constexpr int KB = D / 4 * ESZ;   // K bytes per lane per key
  static constexpr int VB = D / 16 * ESZ;  // V bytes per lane per key
  uint32_t k[2][KB / 4];
  uint32_t v[8][VB / 4];
  int32_t T0;
  bool pvalid[2];
};

template <int D, bool FP8, int WAVES, bool FINAL, int DEPTH>
__global__ __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(2)))
void gqa_decode_kernel(GqaArgs a) {
  using Tile = GqaTile<D, FP8>;
  constexpr int ESZ = Tile::ESZ;
  constexpr int STEPS = D / 32;  // QK MFMA steps
  constexpr int KB = Tile::KB;
  constexpr int VE = D / 16;     // V elements per lane per key (= PV d-tiles)
  constexpr int VB = Tile::VB;
  constexpr int DT = D / 16;     // PV d-tiles
  static_assert(D == 64 || D == 128, "head_dim 64 or 128");

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform, so tile and page indices stay scalar
  const int lane = tid & 63;
  const int g4 = lane >> 4;
  const int li = lane & 15;
  const int g = blockIdx.y;

  int32_t b, split, st, L = 0;
  if (a.dev_split) {  // the split size and the item, from the device's lengths
    gqa_device_item(a, (int32_t)blockIdx.x, b, split, st, L);
    if (!FINAL && blockIdx.x == 0 && blockIdx.y == 0 && tid == 0) *a.ws_st = st;  // for the combine
  } else {
    st = a.split_tiles;
    if ((int32_t)blockIdx.x < a.work_n) {  // the plan's map, from the kernel arguments
      const uint32_t e = a.work[blockIdx.x];
      b = (int32_t)((e & ~kWorkLastSplit) >> 6);
      split = (int32_t)(e & 63u);
    } else {
      locate_work<32>(a.seq_lens, a.B, a.window, st, (int32_t)blockIdx.x, b, split);
    }
  }
  b = __builtin_amdgcn_readfirstlane(b);
  split = __builtin_amdgcn_readfirstlane(split);
  st = __builtin_amdgcn_readfirstlane(st);
  // uniform across the workgroup; a split past the plan's count (a length beyond the plan's bound) is dropped, so no
  // write leaves the workspace
  if (b < 0 || b >= a.B || split >= max(a.max_splits, 1)) return;
  // Query operand: in step s lane (g4, li) holds head li's 8 elements from dim CE (4 c + g4) + w, with CE the
  // elements of a 16-byte cache chunk and 8 s = CE c + w: the dims of the key bytes it feeds in that step.
  constexpr int CE = 16 / ESZ;
  uint32_t qv[STEPS][4];
  {
    const bool live = li < a.group;
    const int32_t h = g * a.group + (live ? li : 0);
    const uint16_t* qp = a.q + ((int64_t)b * a.H + h) * D;
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const int dim = CE * (4 * (8 * s / CE) + g4) + (8 * s) % CE;
      const uint4 w = live ? ld16(qp + dim) : make_uint4(0, 0, 0, 0);
      qv[s][0] = w.x;
      qv[s][1] = w.y;
      qv[s][2] = w.z;
      qv[s][3] = w.w;
    }
  }

  // The row's length by a vector load issued after the query's, so neither the kernel-argument waits nor the query's
  // wait for it: for a full-attention row the split's block-table entries load beside it too. (mbcnt_lo(0, 0) is 0 in
  // every lane, but not provably uniform, so the load stays a vector load.)
  int32_t len_v = L;
  if (!a.dev_split) len_v = a.seq_lens[b + (int32_t)__builtin_amdgcn_mbcnt_lo(0u, 0u)];

  // the stored scales, and the dequantization scales they give (m -> 1 / m for the GPT-OSS multipliers)
  const float kstored = FP8 ? a.k_scale[g] : 1.0f;
  const float vstored = FP8 ? a.v_scale[g] : 1.0f;
  const float kscale = (FP8 && a.mul_scale) ? 1.0f / kstored : kstored;
  const float vscale = (FP8 && a.mul_scale) ? 1.0f / vstored : vstored;
  // the group's sink logits (final outputs only), loaded with the prologue's loads: read after the tile loop, a load
  // there would add a memory round trip to the end of every workgroup
  const float sink_pre = (FINAL && a.sinks && tid < a.group) ? a.sinks[g * a.group + tid] : 0.0f;
  const float qk_scale = a.sm_scale * kscale * kLog2e;
  const int64_t head_stride = (int64_t)a.P * D * ESZ;  // bytes of one (page, head) block
  const int32_t* trow = a.table + (int64_t)b * a.table_stride;
  // Table columns and in-page slots: shifts when the page size is a power of two (uniform).
  const bool p_pow2 = (a.P & (a.P - 1)) == 0;
  const int p_shift = __builtin_ctz((uint32_t)a.P);
  auto column = [&](int32_t key) -> int32_t { return p_pow2 ? key >> p_shift : key / a.P; };
  auto in_page = [&](int32_t key) -> int32_t { return p_pow2 ? key & (a.P - 1) : key % a.P; };
  // The split's block-table entries, when they fit in 256: column col0 + 64 r + lane in pg[r], -1 past the table
  // (then a tile's page is a readlane instead of a scalar load and its wait). Without a window the split's first
  // tile is split * st whatever the row's length, so when a split of st tiles spans at most 256 columns the entries
  // load before the length is known (uniform).
  const int32_t span = (32 % a.P == 0) ? st * 32 / a.P : (st * 32 + a.P - 1) / a.P + 1;
  const bool early = a.window == 0 && span <= 256;
  int32_t col0 = column(split * st * 32);
  int32_t pg[4];
  if (early) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int32_t c = col0 + 64 * r + lane;
      pg[r] = c < a.table_width ? trow[c] : -1;
    }
  }
  L = __builtin_amdgcn_readfirstlane(len_v);
  const KeyRange kr = key_range(L, a.window);
  const int32_t t_first = kr.lo / 32 + split * st;
  const int32_t t_last = min(t_first + st, (kr.hi + 31) / 32);
  bool pre = true;
  if (!early) {
    col0 = column(t_first * 32);
    pre = column(t_last * 32 - 1) - col0 < 256;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int32_t c = col0 + 64 * r + lane;
      pg[r] = (pre && c < a.table_width) ? trow[c] : -1;
    }
  }
  auto table_entry = [&](int32_t col) -> int32_t {
    if (pre) {
      const int32_t c = col - col0;
      const int32_t v = c < 64 ? pg[0] : (c < 128 ? pg[1] : (c < 192 ? pg[2] : pg[3]));
      return __builtin_amdgcn_readlane(v, c & 63);
    }
    return col < a.table_width ? ld_const(trow + col) : -1;
  };

  auto load_tile = [&](Tile& T, int32_t tile) {
    T.T0 = __builtin_amdgcn_readfirstlane(tile * 32);  // uniform: the page lookups below are scalar
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      // page of the half-tile (uniform); an entry outside the table or the pool reads page 0 and is masked
      const int32_t col = column(T.T0 + 16 * hf);
      const int32_t e = table_entry(col);
      T.pvalid[hf] = e >= 0 && (int64_t)e < a.num_blocks;
      const int32_t pgid = T.pvalid[hf] ? e : 0;
      const int64_t blk = ((int64_t)pgid * a.G + g) * head_stride + (int64_t)in_page(T.T0 + 16 * hf) * D * ESZ;
      const uint8_t* kp = a.k_cache + blk + (int64_t)li * D * ESZ + 16 * g4;
#pragma unroll
      for (int c = 0; c < KB / 16; ++c) load_bytes<16>(kp + 64 * c, *reinterpret_cast<uint32_t(*)[4]>(&T.k[hf][4 * c]));
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4)
        load_bytes<VB>(a.v_cache + blk + (int64_t)(4 * g4 + e4) * D * ESZ + VB * li, T.v[4 * hf + e4]);
    }
  };

  float m_ref = kNegBig;  // the reference maximum of this lane's head
  float l_run = 0.0f;     // this lane's share of the softmax sum
  f32x4_t acc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  auto compute_tile = [&](Tile& T) {
    const bool full = T.pvalid[0] && T.pvalid[1] && T.T0 >= kr.lo && T.T0 + 32 <= kr.hi;
    // ---- S^T = K Q^T ----
    f32x4_t sc[2];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      f32x4_t s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < STEPS; ++st) {
        uint32_t op[4];
        if constexpr (FP8) {
          fp8x4_to_bf16x4(T.k[hf][2 * st], op[0], op[1]);
          fp8x4_to_bf16x4(T.k[hf][2 * st + 1], op[2], op[3]);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) op[i] = T.k[hf][4 * st + i];
        }
        s = mfma_16x16x32_bf16(op, qv[st], s);
      }
      sc[hf] = s;
    }
    // ---- mask (boundary tiles only), online softmax ----
    float x[8];
    float tmax = -INFINITY;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int r = 0; r < 4; ++r) x[4 * hf + r] = sc[hf][r] * qk_scale;
    if (!full) {
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int32_t pos = T.T0 + 16 * hf + 4 * g4 + r;
          const bool ok = T.pvalid[hf] && pos >= kr.lo && pos < kr.hi;
          x[4 * hf + r] = ok ? x[4 * hf + r] : -INFINITY;
#pragma unroll
          for (int i = 0; i < VB / 4; ++i) T.v[4 * hf + r][i] = ok ? T.v[4 * hf + r][i] : 0u;
        }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) tmax = fmaxf(tmax, x[i]);
    tmax = max_across_groups(tmax);
    const bool bump = tmax > m_ref + kRescaleSlack;
    if (__any(bump)) {
      const float m_new = bump ? tmax : m_ref;
      const float alpha = __builtin_amdgcn_exp2f(m_ref - m_new);
      m_ref = m_new;
      l_run *= alpha;
#pragma unroll
      for (int t = 0; t < DT; ++t) acc[t] *= alpha;
    }
    float p[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      p[i] = __builtin_amdgcn_exp2f(x[i] - m_ref);
      l_run += p[i];
    }
    const uint32_t pop[4] = {pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]), pack_bf16x2(p[4], p[5]),
                             pack_bf16x2(p[6], p[7])};
    // ---- O^T += V^T P^T, one MFMA per 16-wide d-tile ----
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      uint32_t op[4];
      if constexpr (FP8) {
        // byte t of each key's VB-byte run
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          lo |= ((T.v[e][t >> 2] >> (8 * (t & 3))) & 0xffu) << (8 * e);
          hi |= ((T.v[e + 4][t >> 2] >> (8 * (t & 3))) & 0xffu) << (8 * e);
        }
        fp8x4_to_bf16x4(lo, op[0], op[1]);
        fp8x4_to_bf16x4(hi, op[2], op[3]);
      } else {
        // 16-bit element t of each key's run
#pragma unroll
        for (int pr = 0; pr < 4; ++pr) {
          const uint32_t e0 = (T.v[2 * pr][t >> 1] >> (16 * (t & 1))) & 0xffffu;
          const uint32_t e1 = (T.v[2 * pr + 1][t >> 1] >> (16 * (t & 1))) & 0xffffu;
          op[pr] = e0 | (e1 << 16);
        }
      }
      acc[t] = mfma_16x16x32_bf16(op, pop, acc[t]);
    }
  };

  // The step's own token is attended in-band by the row's last split (and stored). The last split is the row's
  // shortest, so the own token's work delays a workgroup that finishes early rather than one of the row's
  // full-length splits. Its operands (k, v, the slot and the query elements the score needs) load here, with the
  // prologue's loads, so that nothing after the tile loop waits for memory. "Last" is the last split this launch
  // runs for the row: the plan's map counts them (a row's items are consecutive there, splits in order); without a map
  // the items were located from seq_lens, up to the plan's split count. So the own token is attended and stored even
  // when the device's length disagrees with the plan's.
  // (with a map the item's own flag says it, from the entry already loaded)
  const bool own = (int32_t)blockIdx.x < a.work_n ? (a.work[blockIdx.x] & kWorkLastSplit) != 0
                                                   : split == launched_splits(a, b, L, st) - 1;  // uniform
  constexpr int OWN_J = (16 + WAVES - 1) / WAVES;  // query heads per wave in the own token's score
  uint32_t own_kb = 0, own_vb = 0;
  int64_t own_dst = -1;
  float own_q[OWN_J][D / 64];
  if (own) {
    if (tid < D) {
      const int64_t src = ((int64_t)b * a.G + g) * D + tid;
      own_kb = a.k_new[src];
      own_vb = a.v_new[src];
      if (a.new_slots) {
        const int64_t slot = redirect_slot(a.new_slots[b], a.num_blocks * a.P);
        own_dst = (((slot / a.P) * a.G + g) * a.P + slot % a.P) * D + tid;
      }
    }
#pragma unroll
    for (int jj = 0; jj < OWN_J; ++jj) {
      const int j = wave + WAVES * jj;
      const uint16_t* qp = a.q + ((int64_t)b * a.H + g * a.group + min(j, a.group - 1)) * D;
#pragma unroll
      for (int v = 0; v < D / 64; ++v) own_q[jj][v] = bf16_bits_to_f32(qp[lane + 64 * v]);
    }
  }

  // ---- the tile loop: a ring of DEPTH register tiles, DEPTH - 1 of them in flight ahead of the one computed ----
  {
    Tile ring[DEPTH];
    const int32_t t0 = t_first + wave;
#pragma unroll
    for (int i = 0; i < DEPTH - 1; ++i)
      if (t0 + i * WAVES < t_last) load_tile(ring[i], t0 + i * WAVES);
    for (int32_t base = 0;; base += DEPTH) {
      bool done = false;
#pragma unroll
      for (int k = 0; k < DEPTH; ++k) {
        const int32_t cur = t0 + (base + k) * WAVES;
        if (cur >= t_last) {
          done = true;
          break;
        }
        const int32_t nxt = cur + (DEPTH - 1) * WAVES;
        if (nxt < t_last) load_tile(ring[(k + DEPTH - 1) % DEPTH], nxt);
        compute_tile(ring[k]);
      }
      if (done) break;
    }
  }

  // ---- the step's own token (operands loaded before the tile loop) ----
  __shared__ float sm_kn[D], sm_vn[D], sm_sn[16];
  if (own) {
    if (tid < D) {
      const uint32_t kb = own_kb, vb = own_vb;
      const int64_t dst = own_dst;
      float kd, vd;
      if constexpr (FP8) {
        const uint32_t kq = a.mul_scale ? quantize_e4m3fn_mul(kb, kstored) : quantize_e4m3fn(kb, kscale);
        const uint32_t vq = a.mul_scale ? quantize_e4m3fn_mul(vb, vstored) : quantize_e4m3fn(vb, vscale);
        kd = e4m3fn_to_f32(kq) * kscale;
        vd = e4m3fn_to_f32(vq) * vscale;
        if (dst >= 0) {
          a.k_cache[dst] = (uint8_t)kq;
          a.v_cache[dst] = (uint8_t)vq;
        }
      } else {
        kd = bf16_bits_to_f32(kb);
        vd = bf16_bits_to_f32(vb);
        if (dst >= 0) {
          reinterpret_cast<uint16_t*>(a.k_cache)[dst] = (uint16_t)kb;
          reinterpret_cast<uint16_t*>(a.v_cache)[dst] = (uint16_t)vb;
        }
      }
      sm_kn[tid] = kd;
      sm_vn[tid] = vd;
    }
    __syncthreads();
#pragma unroll
    for (int jj = 0; jj < OWN_J; ++jj) {
      const int j = wave + WAVES * jj;  // uniform
      if (j >= a.group) break;
      float s = 0.0f;
#pragma unroll
      for (int v = 0; v < D / 64; ++v) s += own_q[jj][v] * sm_kn[lane + 64 * v];
      s = wave_sum(s);
      if (lane == 0) sm_sn[j] = s * a.sm_scale * kLog2e;
    }
  }

  // ---- merge the waves (and the own token) in LDS; write the output or this split's partial ----
  __shared__ float sm_o[WAVES][16][D + 1];
  __shared__ float sm_sink[16];
  if (FINAL && tid < a.group) sm_sink[tid] = sink_pre;
  __shared__ float sm_m[WAVES][16];
  __shared__ float sm_l[WAVES][16];
  const float l_tot = sum_across_groups(l_run);
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) sm_o[wave][li][VE * (4 * g4 + r) + t] = acc[t][r];
  if (g4 == 0) {
    sm_m[wave][li] = m_ref;
    sm_l[wave][li] = l_tot;
  }
  __syncthreads();
  const int32_t S = a.max_splits;
  for (int idx = tid; idx < a.group * D; idx += 64 * WAVES) {
    const int j = idx / D, d = idx % D;
    const int32_t h = g * a.group + j;
    float M = own ? sm_sn[j] : -INFINITY;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) M = fmaxf(M, sm_m[w][j]);
    float o = 0.0f, l = 0.0f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      const float e = __builtin_amdgcn_exp2f(sm_m[w][j] - M);
      o += e * sm_o[w][j][d];
      l += e * sm_l[w][j];
    }
    o *= vscale;
    if (own) {
      const float e = __builtin_amdgcn_exp2f(sm_sn[j] - M);
      o += e * sm_vn[d];
      l += e;
    }
    if constexpr (FINAL) {
      if (a.sinks) l += __builtin_amdgcn_exp2f(sm_sink[j] * kLog2e - M);
      a.out[((int64_t)b * a.H + h) * D + d] = (uint16_t)f32_to_bf16_bits(o / l);
    } else {
      const int64_t row = ((int64_t)b * S + split) * a.H + h;
      a.ws_o[row * D + d] = o;
      if (d == 0) {
        a.ws_ml[row * 2] = M;
        a.ws_ml[row * 2 + 1] = l;
      }
    }
  }
}

// Merge of a row's splits, one wave per (row, query head): out = sum_s e_s o_s / (sum_s e_s l_s + e_sink), with
// e_s = exp2(m_s - M) and M the maximum over the splits and the sink. Lane s holds split s's weight; lane i holds the
// head dims D / 64 * i .. + D / 64. The partials stream in chunks of 16 splits, each chunk's loads all in flight
// together (the first before the weights are known).
template <int D>
__global__ __launch_bounds__(64) void gqa_combine_kernel(GqaArgs a) {
  constexpr int V = D / 64;
  constexpr int CH = 16;
  const int b = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
  const int32_t S = a.max_splits;
  // The first chunk of partials and every split's (m, l) load before the row's split count is known: they are
  // bounded by the workspace's S splits per row, not by the count, so they do not wait for the seq_lens load. Entries
  // past the count are dropped by selects.
  const int64_t row0 = (int64_t)b * S * a.H + h;
  const float* ob = a.ws_o + row0 * D + V * lane;
  const int64_t sstride = (int64_t)a.H * D;
  float x[CH][V];
#pragma unroll
  for (int k = 0; k < CH; ++k)
#pragma unroll
    for (int v = 0; v < V; ++v) x[k][v] = k < S ? ob[k * sstride + v] : 0.0f;
  float2 ml = make_float2(-INFINITY, 0.0f);
  if (lane < S) ml = *reinterpret_cast<const float2*>(a.ws_ml + (row0 + (int64_t)lane * a.H) * 2);
  const int32_t n = min(launched_splits(a, b, ld_const(a.seq_lens + b), a.dev_split ? *a.ws_st : a.split_tiles), S);
  if (n == 0) return;  // a row with no prior key: the lone-token kernel writes it
  const float m = lane < n ? ml.x : -INFINITY, l = lane < n ? ml.y : 0.0f;
  const float sink = a.sinks ? a.sinks[h] * kLog2e : -INFINITY;
  const float M = fmaxf(wave_max(m), sink);
  const float e = lane < n ? __builtin_amdgcn_exp2f(m - M) : 0.0f;
  const float den = wave_sum(e * l) + (a.sinks ? __builtin_amdgcn_exp2f(sink - M) : 0.0f);
  float o[V];
#pragma unroll
  for (int v = 0; v < V; ++v) o[v] = 0.0f;
  for (int32_t base = 0; base < n; base += CH) {
    if (base > 0) {
#pragma unroll
      for (int k = 0; k < CH; ++k)
#pragma unroll
        for (int v = 0; v < V; ++v) x[k][v] = base + k < n ? ob[(base + k) * sstride + v] : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < CH; ++k) {
      if (base + k < n) {
        const float es = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), base + k));
#pragma unroll
        for (int v = 0; v < V; ++v) o[v] += es * x[k][v];
      }
    }
  }
  const float inv = 1.0f / den;
  uint16_t* dst = a.out + ((int64_t)b * a.H + h) * D + V * lane;
#pragma unroll
  for (int v = 0; v < V; ++v) dst[v] = (uint16_t)f32_to_bf16_bits(o[v] * inv);
}

// Rows with no split at all (seq_len 1) get their output from this pass: only the own token (and the sink).
template <int D, bool FP8>
__global__ __launch_bounds__(128) void gqa_lone_token_kernel(GqaArgs a) {
  const int b = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
  // any split size counts the row's splits as nonzero iff it has a prior key
  if (launched_splits(a, b, a.seq_lens[b], a.split_tiles) > 0) return;
  __shared__ float sm_kn[D], sm_vn[D];
  const float kstored = FP8 ? a.k_scale[g] : 1.0f, vstored = FP8 ? a.v_scale[g] : 1.0f;
  const float kscale = (FP8 && a.mul_scale) ? 1.0f / kstored : kstored;
  const float vscale = (FP8 && a.mul_scale) ? 1.0f / vstored : vstored;
  if (tid < D) {
    const int64_t src = ((int64_t)b * a.G + g) * D + tid;
    const uint32_t kb = a.k_new[src], vb = a.v_new[src];
    int64_t dst = -1;
    if (a.new_slots) {
      const int64_t slot = redirect_slot(a.new_slots[b], a.num_blocks * a.P);
      dst = (((slot / a.P) * a.G + g) * a.P + slot % a.P) * D + tid;
    }
    if constexpr (FP8) {
      const uint32_t kq = a.mul_scale ? quantize_e4m3fn_mul(kb, kstored) : quantize_e4m3fn(kb, kscale);
      const uint32_t vq = a.mul_scale ? quantize_e4m3fn_mul(vb, vstored) : quantize_e4m3fn(vb, vscale);
      sm_kn[tid] = e4m3fn_to_f32(kq) * kscale;
      sm_vn[tid] = e4m3fn_to_f32(vq) * vscale;
      if (dst >= 0) {
        a.k_cache[dst] = (uint8_t)kq;
        a.v_cache[dst] = (uint8_t)vq;
      }
    } else {
      sm_kn[tid] = bf16_bits_to_f32(kb);
      sm_vn[tid] = bf16_bits_to_f32(vb);
      if (dst >= 0) {
        reinterpret_cast<uint16_t*>(a.k_cache)[dst] = (uint16_t)kb;
        reinterpret_cast<uint16_t*>(a.v_cache)[dst] = (uint16_t)vb;
      }
    }
  }
  __syncthreads();
  const int wave = tid >> 6, lane = tid & 63;
  for (int j = wave; j < a.group; j += 2) {
    const int32_t h = g * a.group + j;
    const uint16_t* qp = a.q + ((int64_t)b * a.H + h) * D;
    float s = 0.0f;
    for (int d = lane; d < D; d += 64) s += bf16_bits_to_f32(qp[d]) * sm_kn[d];
    s = wave_sum(s);
    s *= a.sm_scale * kLog2e;
    float M = s, den = 1.0f;
    if (a.sinks) {
      const float sk = a.sinks[h] * kLog2e;
      M = fmaxf(s, sk);
      den = __builtin_amdgcn_exp2f(s - M) + __builtin_amdgcn_exp2f(sk - M);
    }
    const float w = __builtin_amdgcn_exp2f(s - M) / den;
    for (int d = lane; d < D; d += 64) a.out[((int64_t)b * a.H + h) * D + d] = (uint16_t)f32_to_bf16_bits(w * sm_vn[d]);
  }
}

template <int D, bool FP8>
static void launch_gqa(const GqaArgs& a, bool any_lone, hipStream_t s) {
  if (a.n_work > 0) {
    const dim3 grid(a.n_work, a.G);
    // two register tiles per wave whatever the plan's shape (rings of 3 and 4 measured 1% and 2% slower on the cfg2
    // and cfg4 batches: fewer loads outstanding per wave stream faster). Splits of 5 to 64 tiles run on 8 waves, so
    // a wave walks half as many tiles one after the other (cfg4-swa's 5-tile rows 7.98 -> 6.45 us, cfg4's 48-tile
    // splits 24.9 -> 24.3, cfg1's 8-tile splits 12.3 -> 12.1); cfg2's whole 128-tile rows stay on 4 (91 against 94).
    const bool eight = a.split_tiles > 4 && a.split_tiles <= 64;
    if (a.max_splits <= 1) {
      if (eight) hipLaunchKernelGGL((gqa_decode_kernel<D, FP8, 8, true, 2>), grid, dim3(512), 0, s, a);
      else hipLaunchKernelGGL((gqa_decode_kernel<D, FP8, 4, true, 2>), grid, dim3(256), 0, s, a);
    } else {
      if (eight) hipLaunchKernelGGL((gqa_decode_kernel<D, FP8, 8, false, 2>), grid, dim3(512), 0, s, a);
      else hipLaunchKernelGGL((gqa_decode_kernel<D, FP8, 4, false, 2>), grid, dim3(256), 0, s, a);
    }
  }
  if (a.max_splits > 1) hipLaunchKernelGGL((gqa_combine_kernel<D>), dim3(a.B, a.H), dim3(64), 0, s, a);
  if (any_lone) hipLaunchKernelGGL((gqa_lone_token_kernel<D, FP8>), dim3(a.B, a.G), dim3(128), 0, s, a);
}

}  // namespace sna

using namespace sna;

// The library's own split-K workspace for callers that cannot allocate: one array per GPU, resident for the process.
// Host code never passes `scratch` itself to a kernel (its name is a host-side stand-in for the symbol); it passes the
// device address hipGetSymbolAddress gives on each device, looked up once per device with that device current.
static __device__ __align__(256) uint8_t scratch[SNA_NOALLOC_SCRATCH_BYTES];

namespace {

// The checks and launches of one GQA decode, with the split partials in `workspace` (the caller's device memory, or
// the library's scratch array for sna_paged_decode_gqa_noalloc). `what` names the entry point in error messages.
int decode_gqa(const char* what, const void* q, const void* k_cache, const void* v_cache, const float* k_scale,
               const float* v_scale, const int32_t* block_table, int64_t table_stride, int32_t table_width,
               const int32_t* seq_lens, const void* k_new, const void* v_new, const int64_t* new_slots,
               const float* sinks, int32_t window, float sm_scale, void* out, int32_t B, int32_t num_q_heads,
               int32_t num_kv_heads, int32_t head_dim, int32_t page_size, int64_t num_blocks, int32_t cache_dtype,
               const sna_split_plan* plan, void* workspace, int64_t workspace_bytes, void* stream) {
  if (B < 0 || num_q_heads < 1 || num_kv_heads < 1 || num_q_heads % num_kv_heads)
    return fail(SNA_ERR_INVALID_ARGUMENT, "%s: bad head counts (q %d, kv %d)", what, num_q_heads, num_kv_heads);
  const int32_t group = num_q_heads / num_kv_heads;
  if (group > 16)
    return fail(SNA_ERR_UNSUPPORTED, "%s: GQA group %d > 16 (a workgroup covers 16 query heads)", what, group);
  if (head_dim != 64 && head_dim != 128)
    return fail(SNA_ERR_UNSUPPORTED, "%s: head_dim %d (64 or 128 are built)", what, head_dim);
  if (page_size < 16 || page_size % 16)
    return fail(SNA_ERR_UNSUPPORTED, "%s: page_size %d (a multiple of 16 is required)", what, page_size);
  if (cache_dtype != SNA_DTYPE_BF16 && cache_dtype != SNA_DTYPE_FP8_E4M3FN && cache_dtype != SNA_DTYPE_FP8_E4M3FN_MUL)
    return fail(SNA_ERR_INVALID_ARGUMENT, "%s: unknown cache dtype %d", what, cache_dtype);
  if (window < 0 || table_width < 0 || table_stride < table_width || num_blocks < 1 || !(sm_scale > 0.0f))
    return fail(SNA_ERR_INVALID_ARGUMENT, "%s: bad window %d, table %d/%lld, blocks %lld or scale %g", what, window,
                table_width, (long long)table_stride, (long long)num_blocks, (double)sm_scale);
  if (!plan || plan->tile != 32 || plan->split_tiles < 1 || plan->n_work < 0 || plan->max_splits < 0 ||
      plan->batch != B)
    return fail(SNA_ERR_INVALID_ARGUMENT, "%s: missing or foreign split plan (made for %d rows)", what,
                plan ? plan->batch : -1);
  if (const int rc = check_work_map(plan, B, what)) return rc;
  if (plan->device_split && (plan->work_n > 0 || B > kGqaDevSplitRows))
    return fail(SNA_ERR_INVALID_ARGUMENT, "%s: a device-split plan has no item map and at most %d rows (%d)", what,
                kGqaDevSplitRows, B);
  if (B == 0) return SNA_OK;
  const bool fp8 = cache_dtype != SNA_DTYPE_BF16;
  const int64_t need = sna_decode_workspace_bytes(plan, num_q_heads, head_dim);
  if (!q || !k_cache || !v_cache || !block_table || !seq_lens || !k_new || !v_new || !out ||
      (fp8 && (!k_scale || !v_scale)) || (need > 0 && !workspace))
    return fail(SNA_ERR_INVALID_ARGUMENT, "%s: null pointer", what);
  if (!aligned(q, 16) || !aligned(k_cache, 16) || !aligned(v_cache, 16))
    return fail(SNA_ERR_INVALID_ARGUMENT, "%s: q and caches must be 16-byte aligned", what);
  if (workspace_bytes < need)
    return fail(SNA_ERR_WORKSPACE, "%s: workspace of %lld bytes, the plan needs %lld", what,
                (long long)workspace_bytes, (long long)need);
  if (num_q_heads > 65535) return fail(SNA_ERR_INVALID_ARGUMENT, "%s: grid too large", what);

  GqaArgs a;
  a.q = (const uint16_t*)q;
  a.k_cache = (uint8_t*)k_cache;
  a.v_cache = (uint8_t*)v_cache;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  a.mul_scale = cache_dtype == SNA_DTYPE_FP8_E4M3FN_MUL;
  a.table = block_table;
  a.table_stride = table_stride;
  a.table_width = table_width;
  a.seq_lens = seq_lens;
  a.k_new = (const uint16_t*)k_new;
  a.v_new = (const uint16_t*)v_new;
  a.new_slots = new_slots;
  a.sinks = sinks;
  a.B = B;
  a.H = num_q_heads;
  a.G = num_kv_heads;
  a.group = group;
  a.P = page_size;
  a.num_blocks = num_blocks;
  a.window = window;
  a.sm_scale = sm_scale;
  a.split_tiles = plan->split_tiles;
  a.dev_split = plan->device_split;
  a.n_work = plan->n_work;
  a.max_splits = plan->max_splits;
  a.work_n = plan->work_n;
  for (int32_t i = 0; i < plan->work_n; ++i) a.work[i] = plan->work[i];
  if (plan->work_n > 0) {
    for (int32_t r = 0; r < B; ++r) a.row_splits[r] = 0;
    for (int32_t i = 0; i < plan->work_n; ++i) ++a.row_splits[(plan->work[i] & ~kWorkLastSplit) >> 6];
  }
  float* ws = (float*)workspace;
  a.ws_o = need > 0 ? ws : nullptr;
  a.ws_ml = need > 0 ? ws + (int64_t)B * plan->max_splits * num_q_heads * head_dim : nullptr;
  a.ws_st = need > 0 ? (int32_t*)(a.ws_ml + (int64_t)B * plan->max_splits * num_q_heads * 2) : nullptr;
  a.out = (uint16_t*)out;
  // a row with no prior key has no split: the lone-token pass writes it (launched unless the plan rules it out)
  const bool any_lone = !plan->device_split && plan->empty_rows != 0;

  hipStream_t s = (hipStream_t)stream;
  if (head_dim == 128) {
    if (fp8) launch_gqa<128, true>(a, any_lone, s);
    else launch_gqa<128, false>(a, any_lone, s);
  } else {
    if (fp8) launch_gqa<64, true>(a, any_lone, s);
    else launch_gqa<64, false>(a, any_lone, s);
  }
  return check_launch(what);
}

constexpr int64_t kScratchBytes = SNA_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's scratch address, looked up on its first use (SNA_OK), or an error status.
int scratch_address(const char* what, void** ptr) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(SNA_ERR_LAUNCH, "%s: no current device (or device %d past %d)", what, dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(SNA_ERR_LAUNCH, "%s: the scratch array of device %d has no address: %s", what, dev,
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return SNA_OK;
}

}  // namespace

extern "C" int sna_paged_decode_gqa(const void* q, const void* k_cache, const void* v_cache, const float* k_scale,
                                    const float* v_scale, const int32_t* block_table, int64_t table_stride,
                                    int32_t table_width, const int32_t* seq_lens, const void* k_new,
                                    const void* v_new, const int64_t* new_slots, const float* sinks, int32_t window,
                                    float sm_scale, void* out, int32_t B, int32_t num_q_heads, int32_t num_kv_heads,
                                    int32_t head_dim, int32_t page_size, int64_t num_blocks, int32_t cache_dtype,
                                    const sna_split_plan* plan, void* workspace, int64_t workspace_bytes,
                                    void* stream) {
  ApiGuard guard;
  return decode_gqa("paged_decode_gqa", q, k_cache, v_cache, k_scale, v_scale, block_table, table_stride,
                    table_width, seq_lens, k_new, v_new, new_slots, sinks, window, sm_scale, out, B, num_q_heads,
                    num_kv_heads, head_dim, page_size, num_blocks, cache_dtype, plan, workspace, workspace_bytes,
                    stream);
}

extern "C" int sna_paged_decode_gqa_noalloc(const void* q, const void* k_cache, const void* v_cache,
                                            const float* k_scale, const float* v_scale, const int32_t* block_table,
                                            int64_t table_stride, int32_t table_width, const int32_t* seq_lens,
                                            const void* k_new, const void* v_new, const int64_t* new_slots,
                                            const float* sinks, int32_t window, float sm_scale, void* out, int32_t B,
                                            int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                            int32_t page_size, int64_t num_blocks, int32_t cache_dtype,
                                            const sna_split_plan* plan, void* stream) {
  ApiGuard guard;
  const char* what = "paged_decode_gqa_noalloc";
  if (plan && num_q_heads > 0 && head_dim > 0) {
    const int64_t need = sna_decode_workspace_bytes(plan, num_q_heads, head_dim);
    if (need > kScratchBytes)
      return fail(SNA_ERR_WORKSPACE, "%s: the plan's split partials need %lld bytes, past the library's %lld-byte "
                  "scratch (use sna_paged_decode_gqa with a workspace)", what, (long long)need,
                  (long long)kScratchBytes);
  }
  void* ws = nullptr;
  if (const int rc = scratch_address(what, &ws)) return rc;
  return decode_gqa(what, q, k_cache, v_cache, k_scale, v_scale, block_table, table_stride, table_width, seq_lens,
                    k_new, v_new, new_slots, sinks, window, sm_scale, out, B, num_q_heads, num_kv_heads, head_dim,
                    page_size, num_blocks, cache_dtype, plan, ws, kScratchBytes, stream);
}
