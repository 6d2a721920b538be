"""Host logic of the paged store (quashkv_amd.paged.PagedKVStore) on CPU
tensors: page hand-out from the free list, pool growth, page-table width,
release, and the token -> pool-row / V-tile mapping checked entry by entry
against the table."""

import torch

from quashkv_amd.paged import PAGE_SIZES, PagedKVStore

PAGE_TOKENS = PAGE_TOKENS_T = 64


def test_page_sizes():
    assert PAGE_SIZES == (64, 128, 256, 512, 1024, 2048)
    import pytest
    with pytest.raises(ValueError, match="page_tokens"):
        PagedKVStore(1, 1, 64, 2, 3, 1, torch.device("cpu"), page_tokens=96)
    st = PagedKVStore(2, 3, 64, 2, 3, 2, torch.device("cpu"), page_tokens=256)
    st.ensure(300)                               # two 256-token pages each
    assert all(len(p) == 2 for p in st.pages) and st.kpool.shape[2] == 256
    rows = st._rows(250, 10)                     # crosses the page edge at 256
    tiles, j0, n = st._tiles(250, 10)            # tiles 7 (page 0) and 8 (page 1)
    assert (j0, n) == (7, 2)
    for b in range(2):
        for h in range(3):
            for i, t in enumerate(range(250, 260)):
                pg = st.pages[b][t // 256]
                assert int(rows[b, h, i]) == (pg * 3 + h) * 256 + t % 256
            assert int(tiles[b, h, 0]) == (st.pages[b][0] * 3 + h) * 8 + 7
            assert int(tiles[b, h, 1]) == (st.pages[b][1] * 3 + h) * 8 + 0


def test_pages_table_and_rows():
    st = PagedKVStore(B=3, H=2, d=64, mbits=2, vbits=3, num_pages=4, device=torch.device("cpu"),
                      page_tokens=PAGE_TOKENS_T)
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


def test_page_table_host_check():
    import pytest
    from quashkv_amd.paged import check_page_table
    good = torch.tensor([[0, 3, 1], [2, 2, 0]], dtype=torch.int32)
    check_page_table(good, 4)
    for bad in (torch.tensor([[0, 4]], dtype=torch.int32), torch.tensor([[-1, 0]], dtype=torch.int32)):
        with pytest.raises(ValueError, match="page table entries"):
            check_page_table(bad, 4)
    with pytest.raises(ValueError, match="int32"):
        check_page_table(good.long(), 4)
    # the store's own tables always pass (pages come from its pool)
    st = PagedKVStore(3, 2, 64, 2, 3, 1, torch.device("cpu"), page_tokens=64)
    st.ensure(200)
    check_page_table(st.table, st.num_pages)


def test_paged_abi_rejects_empty_pool():
    from quashkv_amd import _native as N
    L = N.lib()
    st = L.qkv_paged_store_append(N.QKV_BF16, 16, None, 1, 1, 64, 128, 2, 3, 16, 16, 16, 16, 16,
                                  16, 16, 16, 16, 16, 1, 64, 0, 0, None)
    assert st == N.QKV_E_INVALID and "num_pages" in L.qkv_last_error().decode()
