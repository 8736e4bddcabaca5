"""Page items of the KV pools, as the reference's prefill-decode transfer moves them. TEST INFRASTRUCTURE ONLY (see
oracle/__init__.py).

A pool's regions are (ptrs, lens, item_lens) from get_contiguous_buf_infos (mem_cache/memory_pool.py:193-202): page p
of region r is the item_lens[r] bytes at ptrs[r] + p * item_lens[r]. A transfer WRITEs item_len bytes from
src_ptr + item_len * src_slot to dst_ptr + item_len * dst_slot (disaggregation/state_transfer.py:9-10); a stripe
into a replicated destination page lands at a block addressed in units of one source item
(disaggregation/dcp_stripes.py:146-161). Here a region is a flat uint8 CPU tensor, an address its byte offset.

The wire layout of pack/unpack (region-major: region r's items from n_pages * (item bytes of the regions before r),
item i at + i * item_lens[r]) is this build's staging format for a transfer buffer; the reference writes items
straight from pool to pool, which copy() restates.
"""

from __future__ import annotations

from typing import List, Sequence

import torch
from torch import Tensor


def capacity(region: Tensor, item_len: int) -> int:
    """Whole items a region holds."""
    return region.numel() // item_len


def item(region: Tensor, item_len: int, page: int) -> Tensor:
    """The item of ``page``: bytes [page * item_len, (page + 1) * item_len) of the region (memory_pool.py:193-202)."""
    return region[page * item_len:(page + 1) * item_len]


def pack(regions: Sequence[Tensor], item_lens: Sequence[int], pages: Sequence[int]) -> Tensor:
    """The items (r, pages[i]) region-major in one uint8 buffer; a page outside region r packs as zeros."""
    parts: List[Tensor] = []
    for reg, il in zip(regions, item_lens):
        for p in pages:
            if 0 <= p < capacity(reg, il):
                parts.append(item(reg, il, p).clone())
            else:
                parts.append(torch.zeros(il, dtype=torch.uint8))
    return torch.cat(parts) if parts else torch.zeros(0, dtype=torch.uint8)


def unpack(wire: Tensor, regions: Sequence[Tensor], item_lens: Sequence[int], pages: Sequence[int]) -> None:
    """Writes a wire buffer of pack's layout into the items (r, pages[i]); a page outside region r is skipped."""
    off = 0
    for reg, il in zip(regions, item_lens):
        for p in pages:
            if 0 <= p < capacity(reg, il):
                item(reg, il, p).copy_(wire[off:off + il])
            off += il


def copy(src: Sequence[Tensor], dst: Sequence[Tensor], item_lens: Sequence[int], src_pages: Sequence[int],
         dst_pages: Sequence[int]) -> None:
    """The transfer's WRITE list: item (r, src_pages[i]) of src to item (r, dst_pages[i]) of dst, both in units of
    item_lens[r] (state_transfer.py:9-10); an item whose source or destination page is outside its region is
    skipped."""
    for s_reg, d_reg, il in zip(src, dst, item_lens):
        for sp, dp in zip(src_pages, dst_pages):
            if 0 <= sp < capacity(s_reg, il) and 0 <= dp < capacity(d_reg, il):
                item(d_reg, il, dp).copy_(item(s_reg, il, sp))
