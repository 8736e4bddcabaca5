// C ABI plumbing: version, error state, split-K planning and the LSE merge of partial results.
#include <algorithm>
#include <cmath>
#include <queue>
#include <vector>

#include "sna_device.h"
#include "sna_host.h"

namespace sna {

char* error_buffer() {
  static thread_local char buf[kErrorBufferBytes];
  return buf;
}

namespace {

int32_t host_splits(int32_t seq_len, int32_t window, int32_t tile, int32_t split_tiles) {
  if (seq_len <= 1) return 0;
  int32_t hi = seq_len - 1;
  int32_t lo = (window > 0 && seq_len - window > 0) ? seq_len - window : 0;
  if (hi <= lo) return 0;
  int32_t t0 = lo / tile, t1 = (hi + tile - 1) / tile;
  return (t1 - t0 + split_tiles - 1) / split_tiles;
}

int32_t host_tiles(int32_t seq_len, int32_t window, int32_t tile) { return host_splits(seq_len, window, tile, 1); }

// The MLA / DSA stream split: every row's key tiles (at least one, so a row with no prior key still has a workgroup
// to attend its own row) laid end to end, cut into n_ctas ranges of equal tile counts. A workgroup runs per CU (the
// kernel's LDS holds one), so n_ctas is the CU count over the head groups, fewer when there are fewer tiles; a sparse workgroup resolves at
// most kMlaMaxSplitKeys indices in LDS, and sparse rows are latency-bound gathers, so a sparse plan aims for
// kSparseTilesPerCta tiles per workgroup (about three per wave: every tile's gathers go out at once). Measured on
// cfg5's 2048-index rows, 11 tiles (~12 workgroups a row) beat 8 (16 a row) by 0.5 us at 16 rows and 0.3 us at 8,
// and tie at 4; 12 tiles and 8 workgroups a row were slower.
constexpr int64_t kSparseTilesPerCta = 11;
int plan_stream(int32_t kind, const int32_t* host_seq_lens, int32_t B, int32_t max_seq_len, int32_t n_keys_per_row,
                int32_t groups, int32_t num_cus, sna_split_plan* plan) {
  plan->device_split = 0;
  if (B > SNA_MAX_PLAN_ROWS)
    return fail(SNA_ERR_UNSUPPORTED, "plan_decode: an MLA / DSA plan holds at most %d rows, not %d (split the batch)",
                SNA_MAX_PLAN_ROWS, B);
  if ((int64_t)B * groups > kStreamMaxCounters)
    return fail(SNA_ERR_UNSUPPORTED, "plan_decode: %d rows x %d head groups exceed the %d merge counters of a launch "
                "(split the batch)", B, groups, kStreamMaxCounters);
  constexpr int32_t kSparseCap = kMlaMaxSplitKeys / 16;  // a sparse range's tiles: its indices resolve in LDS
  if (kind == 1 && !host_seq_lens) {
    // a plan from a bound: the launch cuts its split from the device's lengths, with a workgroup per CU and head
    // group (whole rows while B fits them, equal ranges otherwise); only the workspace and the grid are fixed here
    if (max_seq_len < 1 || max_seq_len - 1 > 65535 * 16)
      return fail(SNA_ERR_UNSUPPORTED, "plan_decode: an MLA bound of %d (1 .. %d keys + 1)", max_seq_len, 65535 * 16);
    const int32_t cus = std::max(1, std::min((num_cus > 0 ? num_cus : 256) / groups, SNA_MAX_CTAS));
    plan->device_split = 1;
    plan->tile = 16;
    plan->batch = B;
    plan->n_ctas = plan->n_work = plan->target_ctas = plan->max_splits = cus;
    plan->total_tiles = 0;
    plan->split_tiles = (max_seq_len - 1 + 15) / 16;
    plan->empty_rows = -1;
    plan->depth = 0;
    plan->work_n = 0;
    plan->wait_polls = kStreamWaitPolls;
    for (int32_t w = 0; w <= SNA_MAX_CTAS; ++w) plan->cta_start[w] = 0;
    for (int32_t w = 0; w < SNA_MAX_CTAS; ++w) plan->cta_row[w] = plan->cta_off[w] = 0;
    for (int32_t b = 0; b < B; ++b) plan->row_keys[b] = max_seq_len - 1;
    return SNA_OK;
  }
  int64_t total = 0, min_pieces = 0;
  int32_t empty = 0, max_tiles = 0;
  for (int32_t b = 0; b < B; ++b) {
    const int32_t keys = kind == 2 ? n_keys_per_row : std::max(host_seq_lens[b] - 1, 0);
    if (kind == 1 && host_seq_lens[b] < 1)
      return fail(SNA_ERR_INVALID_ARGUMENT, "plan_decode: row %d has seq_len %d (at least its new token)", b,
                  host_seq_lens[b]);
    const int32_t tiles = std::max((keys + 15) / 16, 1);
    if (tiles > 65535)
      return fail(SNA_ERR_UNSUPPORTED, "plan_decode: row %d has %d keys, past the stream split's 65535 tiles", b,
                  keys);
    plan->row_keys[b] = keys;
    total += tiles;
    min_pieces += kind == 2 ? (tiles + kSparseCap - 1) / kSparseCap : 1;
    empty += keys == 0;
    max_tiles = std::max(max_tiles, tiles);
  }
  // one round: every 16-head group's workgroups are resident together
  const int32_t cus = std::max(1, std::min((num_cus > 0 ? num_cus : 256) / groups, SNA_MAX_CTAS));
  int64_t n = 0;
  if (total > 0) {
    n = kind == 1 ? std::min<int64_t>(cus, total)
                  : std::min<int64_t>(cus, std::max<int64_t>((total + kSparseTilesPerCta - 1) / kSparseTilesPerCta, 1));
    // a sparse range holds at most kSparseCap tiles: equal ranges need ceil(total / cap) of them, and whole rows
    // (when every row gets a workgroup) need each row's ceil(tiles / cap) pieces
    if (kind == 2) {
      n = std::max<int64_t>(n, (total + kSparseCap - 1) / kSparseCap);
      if (B <= n) n = std::max<int64_t>(n, min_pieces);
    }
    if (n > SNA_MAX_CTAS)
      return fail(SNA_ERR_UNSUPPORTED, "plan_decode: %lld index tiles of %d rows need more than %d workgroups of at "
                  "most %d tiles (split the batch)", (long long)total, B, SNA_MAX_CTAS, kSparseCap);
  }
  // row r's first tile in the global sequence, for the ranges' starting rows
  std::vector<int64_t> first(B + 1, 0);
  for (int32_t b = 0; b < B; ++b) first[b + 1] = first[b] + std::max((plan->row_keys[b] + 15) / 16, 1);
  // The ranges. With a workgroup for every row, rows are apportioned whole: each gets n_b workgroups (at least one),
  // the next one going to the row whose pieces are longest, and its tiles are cut into n_b equal pieces, so no range
  // spans two rows (a second row would restart the tile ring and publish a second partial) and the longest piece is
  // as short as whole pieces allow. With more rows than workgroups the sequence is cut into equal ranges.
  if (n > 0 && B <= n) {
    // every row starts with its least piece count (1; a sparse row: enough pieces of at most kSparseCap tiles)
    std::vector<int32_t> pieces(B, 1);
    int64_t given = 0;
    std::priority_queue<std::pair<double, int32_t>> longest;
    for (int32_t b = 0; b < B; ++b) {
      const int64_t tiles = first[b + 1] - first[b];
      if (kind == 2) pieces[b] = (int32_t)((tiles + kSparseCap - 1) / kSparseCap);
      given += pieces[b];
      longest.push({(double)tiles / pieces[b], b});
    }
    for (int64_t left = n - given; left > 0 && !longest.empty(); --left) {
      const int32_t b = longest.top().second;
      longest.pop();
      const int64_t tiles = first[b + 1] - first[b];
      if (pieces[b] >= tiles) {  // a row never gets more pieces than tiles
        ++left;
        continue;
      }
      ++pieces[b];
      longest.push({(double)tiles / pieces[b], b});
    }
    int64_t w = 0;
    for (int32_t b = 0; b < B; ++b) {
      const int64_t tiles = first[b + 1] - first[b];
      for (int32_t i = 0; i < pieces[b]; ++i, ++w) {
        plan->cta_start[w] = (uint32_t)(first[b] + i * tiles / pieces[b]);
        plan->cta_row[w] = (uint16_t)b;
        plan->cta_off[w] = (uint16_t)(i * tiles / pieces[b]);
      }
    }
    n = w;
    plan->cta_start[n] = (uint32_t)total;
  } else {
    int32_t row = 0;
    for (int64_t w = 0; w <= n; ++w) {
      const int64_t g = w * total / std::max<int64_t>(n, 1);
      plan->cta_start[w] = (uint32_t)g;
      if (w == n) break;
      while (row + 1 < B && first[row + 1] <= g) ++row;
      plan->cta_row[w] = (uint16_t)row;
      plan->cta_off[w] = (uint16_t)(g - first[row]);
    }
  }
  int32_t widest = 0;
  // the most workgroups one row spans (the merge's partial count)
  for (int32_t b = 0, w = 0; b < B && n > 0; ++b) {
    while (w + 1 < n && (int64_t)plan->cta_start[w + 1] <= first[b]) ++w;
    int32_t w_end = w;
    while (w_end + 1 < n && (int64_t)plan->cta_start[w_end + 1] < first[b + 1]) ++w_end;
    widest = std::max(widest, w_end - w + 1);
  }
  int64_t longest_range = 0;
  for (int64_t w = 0; w < n; ++w)
    longest_range = std::max<int64_t>(longest_range, (int64_t)plan->cta_start[w + 1] - plan->cta_start[w]);
  plan->split_tiles = (int32_t)longest_range;
  plan->n_work = (int32_t)n;
  plan->tile = 16;
  plan->target_ctas = cus;
  plan->max_splits = widest;
  plan->batch = B;
  plan->empty_rows = empty;
  plan->depth = 0;
  plan->work_n = 0;
  plan->n_ctas = (int32_t)n;
  plan->total_tiles = (int32_t)total;
  plan->wait_polls = kStreamWaitPolls;
  (void)max_tiles;
  return SNA_OK;
}

}  // namespace

// ---- LSE merge of partials (decode-context-parallel style) ----
__global__ __launch_bounds__(256) void lse_combine_kernel(const float* __restrict__ o_parts,
                                                          const float* __restrict__ lse_parts, int32_t n_parts,
                                                          int64_t n_rows, int32_t dim, uint16_t* __restrict__ out,
                                                          float* __restrict__ lse_out) {
  const int64_t row = blockIdx.x;
  float m = -INFINITY;
  for (int32_t i = 0; i < n_parts; ++i) m = fmaxf(m, lse_parts[(int64_t)i * n_rows + row]);
  float den = 0.0f;
  for (int32_t i = 0; i < n_parts; ++i) {
    const float l = lse_parts[(int64_t)i * n_rows + row];
    den += (m == -INFINITY) ? 0.0f : expf(l - m);
  }
  const float lse = (m == -INFINITY || den == 0.0f) ? -INFINITY : m + logf(den);
  for (int32_t d = threadIdx.x; d < dim; d += blockDim.x) {
    float acc = 0.0f;
    if (lse != -INFINITY) {
      for (int32_t i = 0; i < n_parts; ++i) {
        const float l = lse_parts[(int64_t)i * n_rows + row];
        if (l == -INFINITY) continue;
        acc += expf(l - lse) * o_parts[((int64_t)i * n_rows + row) * dim + d];
      }
    }
    out[row * dim + d] = (uint16_t)f32_to_bf16_bits(acc);
  }
  if (lse_out && threadIdx.x == 0) lse_out[row] = lse;
}

}  // namespace sna

using namespace sna;

extern "C" {

int sna_version(void) { return 101; }

const char* sna_last_error(void) { return error_buffer(); }

int sna_plan_decode(int32_t kind, const int32_t* host_seq_lens, int32_t B, int32_t max_seq_len, int32_t window,
                    int32_t n_keys_per_row, int32_t ctas_per_item, int32_t num_cus, sna_split_plan* plan) {
  ApiGuard guard;
  const int32_t gqa_depth = plan ? plan->depth : 0;  // a caller may preset the plan shape it wants (2 or 3)
  if (!plan) return fail(SNA_ERR_INVALID_ARGUMENT, "plan_decode: null plan");
  plan->device_split = 0;
  if (kind < 0 || kind > 2) return fail(SNA_ERR_INVALID_ARGUMENT, "plan_decode: unknown kind %d", kind);
  if (B < 0 || ctas_per_item < 1 || window < 0)
    return fail(SNA_ERR_INVALID_ARGUMENT, "plan_decode: bad arguments (B %d, ctas_per_item %d, window %d)", B,
                ctas_per_item, window);
  if (kind == 2 && n_keys_per_row < 0)
    return fail(SNA_ERR_INVALID_ARGUMENT, "plan_decode: negative index count %d", n_keys_per_row);
  if (kind != 2 && !host_seq_lens && max_seq_len < 0)
    return fail(SNA_ERR_INVALID_ARGUMENT, "plan_decode: need host seq_lens or max_seq_len >= 0");
  if (kind != 0)
    return plan_stream(kind, host_seq_lens, B, max_seq_len, n_keys_per_row, ctas_per_item, num_cus, plan);
  const int32_t tile = kind == 0 ? 32 : 16;
  const int32_t waves = 4;
  const int32_t cus = num_cus > 0 ? num_cus : 256;
  const int32_t win = kind == 2 ? 0 : window;
  // A plan from a bound holds every length up to it. With a window, the tiles a row spans depend on where its window
  // starts inside a tile (periodic in the length, period `tile`), so the bound takes the most tiles of any length in
  // its last two periods; below the window the count only grows with the length.
  int32_t bound_tiles = 0;
  if (kind != 2 && !host_seq_lens)
    for (int32_t L = std::max(1, max_seq_len - 2 * tile); L <= max_seq_len; ++L)
      bound_tiles = std::max(bound_tiles, host_tiles(L, win, tile));
  auto tiles_of = [&](int32_t b) -> int32_t {
    if (kind == 2) return host_tiles(n_keys_per_row + 1, 0, tile);  // the index list as "prior keys" + the own row
    return host_seq_lens ? host_tiles(host_seq_lens[b], win, tile) : bound_tiles;
  };
  auto splits_of_row = [&](int32_t b, int32_t st) -> int32_t { return (tiles_of(b) + st - 1) / st; };
  int64_t total_tiles = 0;
  int32_t max_tiles = 0;
  for (int32_t b = 0; b < B; ++b) {
    int32_t t = tiles_of(b);
    total_tiles += t;
    max_tiles = std::max(max_tiles, t);
  }
  // GQA plan shape: one round of two workgroups per CU (3) when there is enough work to fill the chip with long
  // splits; several rounds of smaller splits (2) keep small launches short.
  const int32_t depth = gqa_depth > 0 ? gqa_depth : (total_tiles * ctas_per_item >= (int64_t)cus * 32 ? 3 : 2);
  // Resident workgroups the launch aims for, and whether it must fit them in one round. GQA with the deep ring holds
  // two 4-wave workgroups per CU and runs one round; the shallow ring holds about three and runs a few rounds. The
  // MLA kernels hold one per CU (their register and LDS budget) and run one round.
  const bool one_round = kind != 0 || depth >= 3;
  const int64_t target = kind == 0 ? (int64_t)cus * (depth >= 3 ? 2 : 8) : (int64_t)cus;
  const int64_t items_target = std::max<int64_t>(1, target / ctas_per_item);
  int32_t split_tiles = (int32_t)std::max<int64_t>(waves, (total_tiles + items_target - 1) / items_target);
  // short rows (a sliding window, a few pages) stay whole: one split, no combine pass
  split_tiles = std::max(split_tiles, std::min(max_tiles, 2 * waves));
  // A MLA split's row ids live in the kernel's LDS, which caps it at kMlaMaxSplitTiles tiles.
  constexpr int32_t kMlaMaxSplitTiles = kMlaMaxSplitKeys / 16;
  const int32_t cap = kind != 0 ? kMlaMaxSplitTiles : std::max(max_tiles, waves);
  split_tiles = std::min(split_tiles, cap);
  if (one_round) {
    // grow the split until the item count fits the resident target, so no workgroup waits for a second round
    while (split_tiles < cap) {
      int64_t n = 0;
      for (int32_t b = 0; b < B; ++b) n += splits_of_row(b, split_tiles);
      if (n * ctas_per_item <= target) break;
      split_tiles = std::min(split_tiles + 1, cap);
    }
  }
  // the combine passes hold at most kMaxSplits weights per row: grow the split until every row fits
  while (true) {
    int32_t worst = 0;
    for (int32_t b = 0; b < B; ++b) worst = std::max(worst, splits_of_row(b, split_tiles));
    if (worst <= kMaxSplits) break;
    split_tiles = std::max(split_tiles + 1, (max_tiles + kMaxSplits - 1) / kMaxSplits);
  }
  if (kind != 0 && split_tiles * tile > kMlaMaxSplitKeys)
    return fail(SNA_ERR_UNSUPPORTED, "plan_decode: a row of %d tiles needs splits beyond the MLA kernel's capacity",
                max_tiles);
  int64_t n_work = 0;
  int32_t max_splits = 0, empty = 0;
  for (int32_t b = 0; b < B; ++b) {
    const int32_t n = splits_of_row(b, split_tiles);
    n_work += n;
    max_splits = std::max(max_splits, n);
    empty += n == 0;
  }
  if (n_work > INT32_MAX / 2 || (int64_t)B * max_splits > INT32_MAX / 2)
    return fail(SNA_ERR_INVALID_ARGUMENT, "plan_decode: too many splits");
  plan->split_tiles = split_tiles;
  plan->n_work = (int32_t)n_work;
  plan->tile = tile;
  plan->target_ctas = (int32_t)target;
  plan->max_splits = max_splits;
  plan->batch = B;
  if (kind == 0 && !host_seq_lens && B <= kGqaDevSplitRows && bound_tiles <= kGqaDevSplitMaxTiles) {
    // A GQA plan from a bound splits on the device: every launch sizes its splits from the device's lengths by the
    // one-round rule above to fit the items the bound's own split runs, and gives every row a split (a row with no
    // prior key attends its own token there: no lone-token pass). A split holds at least 4 tiles and at least
    // min(longest row, 8), so a row of up to 8 tiles is one split and a longer one at most ceil(tiles / 8); and as
    // every other row takes an item, a row gets at most n_work - B + 1 (one, when the bound's split is whole rows).
    plan->device_split = 1;
    plan->n_work = (int32_t)std::max<int64_t>(n_work, B);
    plan->max_splits = std::min(bound_tiles <= 8 ? 1 : std::min(kMaxSplits, (bound_tiles + 7) / 8),
                                plan->n_work - B + 1);
  }
  // a plan from a bound cannot know which rows are only their new token (a device split gives every row a split)
  plan->empty_rows = plan->device_split ? 0 : (kind != 2 && !host_seq_lens) ? -1 : empty;
  plan->depth = kind == 0 ? depth : 0;
  // the item -> (row, split) map, when the lengths are exact and the items fit it (the order locate_work finds)
  plan->work_n = 0;
  if (kind != 2 && host_seq_lens && n_work <= SNA_MAX_WORK_MAP && B <= SNA_MAX_WORK_MAP) {
    int32_t i = 0;
    for (int32_t b = 0; b < B; ++b)
      for (int32_t s = 0, n = splits_of_row(b, split_tiles); s < n; ++s)
        plan->work[i++] = ((uint32_t)b << 6) | s | (s == n - 1 ? kWorkLastSplit : 0u);
    plan->work_n = i;
  }
  return SNA_OK;
}

int sna_check_decode_operands(const int64_t* seq_lens, const int32_t* block_table, int64_t table_stride,
                              int32_t table_width, const int64_t* new_slots, const int32_t* active, int32_t B,
                              int32_t page_size, int64_t num_blocks) {
  ApiGuard guard;
  if (B < 0 || page_size < 1 || num_blocks < 1 || table_width < 0 || table_stride < table_width)
    return fail(SNA_ERR_INVALID_ARGUMENT, "check_decode_operands: bad sizes (B %d, page %d, blocks %lld, table %d/%lld)",
                B, page_size, (long long)num_blocks, table_width, (long long)table_stride);
  if (B == 0) return SNA_OK;
  if (!seq_lens || (table_width > 0 && !block_table))
    return fail(SNA_ERR_INVALID_ARGUMENT, "check_decode_operands: null pointer");
  const int64_t pool_slots = num_blocks * page_size;
  // A row is live by its flag; without flags, unless it is a padding row: its own token only (seq_len 1) written to
  // the reserved page 0 or outside the pool (redirected to slot 0).
  auto in_pool = [&](int64_t slot) { return slot >= page_size && slot < pool_slots; };
  auto live = [&](int32_t b) { return active ? active[b] != 0 : (seq_lens[b] > 1 || in_pool(new_slots[b])); };
  for (int32_t b = 0; b < B; ++b) {
    const int64_t L = seq_lens[b];
    if (L < 1) return fail(SNA_ERR_INVALID_ARGUMENT, "row %d: seq_len %lld (a decode row holds at least its new token)",
                           b, (long long)L);
    if (L > INT32_MAX)
      return fail(SNA_ERR_INVALID_ARGUMENT, "row %d: position %lld exceeds the kernels' int32 positions", b,
                  (long long)(L - 1));
    const int64_t pages = (L + page_size - 1) / page_size;
    if (pages > table_width)
      return fail(SNA_ERR_INVALID_ARGUMENT, "row %d: %lld tokens span %lld pages, the block table holds %d", b,
                  (long long)L, (long long)pages, table_width);
    const int32_t* row = block_table + (int64_t)b * table_stride;
    for (int64_t j = 0; j < pages; ++j)
      if (row[j] < 0 || row[j] >= num_blocks)
        return fail(SNA_ERR_INVALID_ARGUMENT, "row %d: table column %lld holds page %d, outside the pool's %lld pages "
                    "(the row's pages must cover its %lld tokens)", b, (long long)j, row[j], (long long)num_blocks,
                    (long long)L);
    if (!new_slots || !live(b)) continue;
    const int64_t slot = new_slots[b];
    if (!in_pool(slot))
      return fail(SNA_ERR_INVALID_ARGUMENT, "row %d: live row's new slot %lld is %s (the write would go to the reserved "
                  "slot 0 and the token be lost)", b, (long long)slot,
                  slot < 0 || slot >= pool_slots ? "outside the pool" : "on the reserved page 0");
    if (slot % page_size != (L - 1) % page_size)
      return fail(SNA_ERR_INVALID_ARGUMENT, "row %d: new slot %lld disagrees with position %lld (page %d)", b,
                  (long long)slot, (long long)(L - 1), page_size);
    if (slot / page_size != row[(L - 1) / page_size])
      return fail(SNA_ERR_INVALID_ARGUMENT, "row %d: new slot %lld is on page %lld, the row's last page is %d", b,
                  (long long)slot, (long long)(slot / page_size), row[(L - 1) / page_size]);
  }
  if (new_slots) {
    std::vector<int64_t> written;
    written.reserve(B);
    for (int32_t b = 0; b < B; ++b)
      if (live(b)) written.push_back(new_slots[b]);
    std::sort(written.begin(), written.end());
    for (size_t i = 1; i < written.size(); ++i)
      if (written[i] == written[i - 1])
        return fail(SNA_ERR_INVALID_ARGUMENT, "two live decode rows write slot %lld", (long long)written[i]);
  }
  return SNA_OK;
}

int64_t sna_decode_workspace_bytes(const sna_split_plan* plan, int32_t num_q_heads, int32_t head_dim_v) {
  if (!plan || num_q_heads < 1 || head_dim_v < 1) return 0;
  if (plan->tile == 16) {  // MLA / DSA stream split: counters, then two partial slots per workgroup
    if (plan->n_ctas < 1) return 0;
    return kStreamCounterBytes +
           2ll * plan->n_ctas * num_q_heads * ((int64_t)head_dim_v + 2) * (int64_t)sizeof(float);
  }
  if (plan->max_splits <= 1) return 0;
  // partials, then (a device split) the launch's split size for its combine, in a 256-byte line
  return (int64_t)plan->batch * plan->max_splits * num_q_heads * ((int64_t)head_dim_v + 2) * (int64_t)sizeof(float) +
         (plan->device_split ? 256 : 0);
}

int sna_lse_combine(const float* o_parts, const float* lse_parts, int32_t n_parts, int64_t n_rows, int32_t dim,
                    void* out, float* lse_out, void* stream) {
  ApiGuard guard;
  if (n_parts < 1 || n_rows < 0 || dim < 1)
    return fail(SNA_ERR_INVALID_ARGUMENT, "lse_combine: bad sizes (parts %d, rows %lld, dim %d)", n_parts,
                (long long)n_rows, dim);
  if (n_rows == 0) return SNA_OK;
  if (!o_parts || !lse_parts || !out) return fail(SNA_ERR_INVALID_ARGUMENT, "lse_combine: null pointer");
  if (n_rows > INT32_MAX) return fail(SNA_ERR_INVALID_ARGUMENT, "lse_combine: too many rows");
  hipLaunchKernelGGL(lse_combine_kernel, dim3((unsigned)n_rows), dim3(256), 0, (hipStream_t)stream, o_parts,
                     lse_parts, n_parts, n_rows, dim, (uint16_t*)out, lse_out);
  return check_launch("lse_combine");
}

}  // extern "C"
