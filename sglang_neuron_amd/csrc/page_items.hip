// Page items of the KV pools on the GPU: the unit a prefill-decode (PD) transfer moves. A pool exposes its regions
// (one per layer's K or V buffer, or per layer's row buffer) as (ptrs, lens, item_lens): page p of region r is the
// item_lens[r] bytes at ptrs[r] + p * item_lens[r], and a transfer writes whole items, source page to destination
// page.
//   reference: mem_cache/memory_pool.py:193-202 (get_contiguous_buf_infos, the item addressing);
//   disaggregation/state_transfer.py:9-10 (a transfer WRITEs item_len bytes from src_ptr + item_len * src_slot to
//   dst_ptr + item_len * dst_slot); disaggregation/dcp_stripes.py:146-161 (stripes land in destination blocks in
//   units of one source item).
//
// Three moves over one kernel:
//   pack:    the items (region r, pages[i]) into a contiguous wire buffer, region-major: region r's items start at
//            n_pages * (item bytes of the regions before r), item i at + i * item_lens[r];
//   unpack:  a wire buffer of that layout into the items (region r, pages[i]);
//   copy:    item (r, src_pages[i]) of the source regions to item (r, dst_pages[i]) of the destination regions
//            (the transfer's WRITE list on one GPU).
// One workgroup per (item, region), 16-byte non-temporal loads and stores (every byte is touched once); HBM-bound:
// 2 bytes of traffic per byte moved.

#include <cstring>
#include <vector>

#include "sna_device.h"
#include "sna_host.h"

namespace sna {

// regions per launch: the region table travels in the kernel arguments (96 x 32 B, under their 4 KB)
constexpr int kItemRegions = 96;

struct ItemRegion {
  uint64_t src, dst;         // base addresses of the item arrays read and written
  int32_t item;              // bytes per item (a multiple of 16)
  int32_t src_cap, dst_cap;  // items in each array
  int32_t pad;
};
static_assert(sizeof(ItemRegion) == 32, "a 32-byte region record");

struct PageItemsArgs {
  ItemRegion r[kItemRegions];
  const int32_t* src_pages;  // [n_pages] the item read, or null: item i
  const int32_t* dst_pages;  // [n_pages] the item written, or null: item i
  int32_t zero_invalid;      // an item whose source page is outside its array is written as zeros (pack)
};

__global__ __launch_bounds__(256) void page_items_kernel(PageItemsArgs a) {
  const int64_t i = blockIdx.x;
  const ItemRegion g = a.r[blockIdx.y];
  const int64_t sp = a.src_pages ? (int64_t)a.src_pages[i] : i;
  const int64_t dp = a.dst_pages ? (int64_t)a.dst_pages[i] : i;
  if (dp < 0 || dp >= g.dst_cap) return;  // (uniform) nowhere to write
  typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
  u32x4_t* dst = reinterpret_cast<u32x4_t*>(g.dst + (uint64_t)dp * (uint64_t)g.item);
  const int32_t n = g.item >> 4;  // 16-byte vectors
  if (sp < 0 || sp >= g.src_cap) {  // (uniform)
    if (a.zero_invalid) {
      const u32x4_t z = {0u, 0u, 0u, 0u};
      for (int32_t v = threadIdx.x; v < n; v += 256) __builtin_nontemporal_store(z, dst + v);
    }
    return;
  }
  const u32x4_t* src = reinterpret_cast<const u32x4_t*>(g.src + (uint64_t)sp * (uint64_t)g.item);
  // four vectors in flight per lane before the first store
  int32_t v = threadIdx.x;
  for (; v + 3 * 256 < n; v += 4 * 256) {
    u32x4_t x[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) x[u] = __builtin_nontemporal_load(src + v + u * 256);
#pragma unroll
    for (int u = 0; u < 4; ++u) __builtin_nontemporal_store(x[u], dst + v + u * 256);
  }
  for (; v < n; v += 256) __builtin_nontemporal_store(__builtin_nontemporal_load(src + v), dst + v);
}

namespace {

// Validates the host region description; *total_item_bytes = the bytes of one page over all regions.
int check_regions(const char* what, const uint64_t* ptrs, const int64_t* lens, const int64_t* item_lens,
                  int32_t n_regions, int64_t* total_item_bytes) {
  int64_t total = 0;
  for (int32_t r = 0; r < n_regions; ++r) {
    if (!ptrs[r] || item_lens[r] <= 0 || item_lens[r] % 16 != 0 || ptrs[r] % 16 != 0 || lens[r] < 0 ||
        item_lens[r] > 0x7fffffffLL || lens[r] / item_lens[r] > 0x7fffffffLL)
      return fail(SNA_ERR_INVALID_ARGUMENT,
                  "%s: region %d (address %llx, %lld bytes, items of %lld bytes): the address and the item size "
                  "must be non-zero multiples of 16, items under 2 GiB and fewer than 2^31 of them",
                  what, r, (unsigned long long)ptrs[r], (long long)lens[r], (long long)item_lens[r]);
    total += item_lens[r];
  }
  if (total_item_bytes) *total_item_bytes = total;
  return SNA_OK;
}

// Launches the moves in batches of kItemRegions regions; fill(args, r0, nr) fills the batch's region table.
template <class Fill>
int launch_items(const char* what, int32_t n_regions, int64_t n_pages, const int32_t* src_pages,
                 const int32_t* dst_pages, int zero_invalid, hipStream_t stream, Fill fill) {
  if (n_pages > 0x7fffffffLL) return fail(SNA_ERR_INVALID_ARGUMENT, "%s: %lld pages exceed the grid", what,
                                          (long long)n_pages);
  const int32_t batches = (n_regions + kItemRegions - 1) / kItemRegions;
  const int32_t per = (n_regions + batches - 1) / batches;  // even batches
  for (int32_t r0 = 0; r0 < n_regions; r0 += per) {
    const int32_t nr = n_regions - r0 < per ? n_regions - r0 : per;
    PageItemsArgs a;
    memset(&a, 0, sizeof(a));
    fill(a, r0, nr);
    a.src_pages = src_pages;
    a.dst_pages = dst_pages;
    a.zero_invalid = zero_invalid;
    hipLaunchKernelGGL(page_items_kernel, dim3((unsigned)n_pages, (unsigned)nr), dim3(256), 0, stream, a);
  }
  return check_launch(what);
}

}  // namespace
}  // namespace sna

using namespace sna;

int64_t sna_page_items_wire_bytes(const int64_t* item_lens, int32_t n_regions, int64_t n_pages) {
  if (!item_lens || n_regions < 0 || n_pages < 0) return -1;
  int64_t t = 0;
  for (int32_t r = 0; r < n_regions; ++r) t += item_lens[r];
  return t * n_pages;
}

int sna_page_items_pack(const uint64_t* region_ptrs, const int64_t* region_lens, const int64_t* item_lens,
                        int32_t n_regions, const int32_t* pages, int64_t n_pages, void* wire, int64_t wire_bytes,
                        void* stream) {
  ApiGuard guard;
  if (n_regions < 0 || n_pages < 0)
    return fail(SNA_ERR_INVALID_ARGUMENT, "page_items_pack: %d regions, %lld pages", n_regions, (long long)n_pages);
  if (n_regions == 0 || n_pages == 0) return SNA_OK;
  if (!region_ptrs || !region_lens || !item_lens || !pages || !wire)
    return fail(SNA_ERR_INVALID_ARGUMENT, "page_items_pack: null pointer");
  int64_t per_page = 0;
  if (int rc = check_regions("page_items_pack", region_ptrs, region_lens, item_lens, n_regions, &per_page)) return rc;
  if (!aligned(wire, 16)) return fail(SNA_ERR_INVALID_ARGUMENT, "page_items_pack: the wire buffer must be 16-B aligned");
  if (wire_bytes < per_page * n_pages)
    return fail(SNA_ERR_WORKSPACE, "page_items_pack: a wire buffer of %lld bytes, the items need %lld",
                (long long)wire_bytes, (long long)(per_page * n_pages));
  std::vector<int64_t> off(n_regions);
  int64_t acc = 0;
  for (int32_t r = 0; r < n_regions; ++r) off[r] = acc, acc += item_lens[r] * n_pages;
  return launch_items("page_items_pack", n_regions, n_pages, pages, nullptr, 1, (hipStream_t)stream,
                      [&](PageItemsArgs& a, int32_t r0, int32_t nr) {
                        for (int32_t j = 0; j < nr; ++j) {
                          const int32_t r = r0 + j;
                          a.r[j] = {region_ptrs[r], (uint64_t)wire + (uint64_t)off[r], (int32_t)item_lens[r],
                                    (int32_t)(region_lens[r] / item_lens[r]), (int32_t)n_pages, 0};
                        }
                      });
}

int sna_page_items_unpack(const void* wire, int64_t wire_bytes, const uint64_t* region_ptrs,
                          const int64_t* region_lens, const int64_t* item_lens, int32_t n_regions,
                          const int32_t* pages, int64_t n_pages, void* stream) {
  ApiGuard guard;
  if (n_regions < 0 || n_pages < 0)
    return fail(SNA_ERR_INVALID_ARGUMENT, "page_items_unpack: %d regions, %lld pages", n_regions, (long long)n_pages);
  if (n_regions == 0 || n_pages == 0) return SNA_OK;
  if (!region_ptrs || !region_lens || !item_lens || !pages || !wire)
    return fail(SNA_ERR_INVALID_ARGUMENT, "page_items_unpack: null pointer");
  int64_t per_page = 0;
  if (int rc = check_regions("page_items_unpack", region_ptrs, region_lens, item_lens, n_regions, &per_page))
    return rc;
  if (!aligned(wire, 16))
    return fail(SNA_ERR_INVALID_ARGUMENT, "page_items_unpack: the wire buffer must be 16-B aligned");
  if (wire_bytes < per_page * n_pages)
    return fail(SNA_ERR_INVALID_ARGUMENT, "page_items_unpack: a wire buffer of %lld bytes, the items need %lld",
                (long long)wire_bytes, (long long)(per_page * n_pages));
  std::vector<int64_t> off(n_regions);
  int64_t acc = 0;
  for (int32_t r = 0; r < n_regions; ++r) off[r] = acc, acc += item_lens[r] * n_pages;
  return launch_items("page_items_unpack", n_regions, n_pages, nullptr, pages, 0, (hipStream_t)stream,
                      [&](PageItemsArgs& a, int32_t r0, int32_t nr) {
                        for (int32_t j = 0; j < nr; ++j) {
                          const int32_t r = r0 + j;
                          a.r[j] = {(uint64_t)wire + (uint64_t)off[r], region_ptrs[r], (int32_t)item_lens[r],
                                    (int32_t)n_pages, (int32_t)(region_lens[r] / item_lens[r]), 0};
                        }
                      });
}

int sna_page_items_copy(const uint64_t* src_ptrs, const int64_t* src_lens, const uint64_t* dst_ptrs,
                        const int64_t* dst_lens, const int64_t* item_lens, int32_t n_regions,
                        const int32_t* src_pages, const int32_t* dst_pages, int64_t n_pages, void* stream) {
  ApiGuard guard;
  if (n_regions < 0 || n_pages < 0)
    return fail(SNA_ERR_INVALID_ARGUMENT, "page_items_copy: %d regions, %lld pages", n_regions, (long long)n_pages);
  if (n_regions == 0 || n_pages == 0) return SNA_OK;
  if (!src_ptrs || !src_lens || !dst_ptrs || !dst_lens || !item_lens || !src_pages || !dst_pages)
    return fail(SNA_ERR_INVALID_ARGUMENT, "page_items_copy: null pointer");
  if (int rc = check_regions("page_items_copy", src_ptrs, src_lens, item_lens, n_regions, nullptr)) return rc;
  if (int rc = check_regions("page_items_copy", dst_ptrs, dst_lens, item_lens, n_regions, nullptr)) return rc;
  return launch_items("page_items_copy", n_regions, n_pages, src_pages, dst_pages, 0, (hipStream_t)stream,
                      [&](PageItemsArgs& a, int32_t r0, int32_t nr) {
                        for (int32_t j = 0; j < nr; ++j) {
                          const int32_t r = r0 + j;
                          a.r[j] = {src_ptrs[r], dst_ptrs[r], (int32_t)item_lens[r],
                                    (int32_t)(src_lens[r] / item_lens[r]), (int32_t)(dst_lens[r] / item_lens[r]), 0};
                        }
                      });
}
