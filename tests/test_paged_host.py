"""Host logic of the paged store (quashkv_amd.paged.PagedKVStore) on CPU
tensors: page hand-out from the free list, pool growth, page-table width,
release, and the token -> pool-row / V-tile mapping checked entry by entry
against the table."""

import torch

from quashkv_amd.paged import PAGE_TOKENS, PagedKVStore


def test_pages_table_and_rows():
    st = PagedKVStore(B=3, H=2, d=64, mbits=2, vbits=3, num_pages=4, device=torch.device("cpu"))
    st.free = [3, 1, 0, 2]
    st.ensure(1)                                 # one page per sequence
    assert st.pages == [[3], [1], [0]] and st.free == [2]
    st.ensure(130)                               # three pages each: pool grows
    assert st.num_pages >= 9 and all(len(p) == 3 for p in st.pages)
    assert st.pages_per_seq >= 3
    ids = sum(st.pages, [])
    assert len(set(ids)) == 9 and sorted(ids + st.free) == list(range(st.num_pages))
    tab = st.table
    for b in range(3):
        assert tab[b, :3].tolist() == st.pages[b]
    rows = st._rows(60, 10)                      # crosses the first page edge
    for b in range(3):
        for h in range(2):
            for i, t in enumerate(range(60, 70)):
                pg = st.pages[b][t // PAGE_TOKENS]
                assert int(rows[b, h, i]) == (pg * 2 + h) * PAGE_TOKENS + t % PAGE_TOKENS
    tiles, j0, n = st._tiles(60, 10)             # tiles 1 and 2
    assert (j0, n) == (1, 2)
    for b in range(3):
        for h in range(2):
            for i, j in enumerate((1, 2)):
                pg = st.pages[b][j // 2]
                assert int(tiles[b, h, i]) == (pg * 2 + h) * 2 + j % 2
    st.release()
    assert not any(st.pages) and len(st.free) == st.num_pages
    st.ensure(64)                                # released pages are handed out again
    assert len(set(sum(st.pages, []))) == 3 and len(st.free) == st.num_pages - 3
