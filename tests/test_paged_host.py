"""Host side of the paged caches (no GPU): PageTable's page accounting on CPU tensors.

No counterpart in the reference (contiguous caches only; paged KV is its future work,
README.md:121-123)."""
import pytest
import torch

from exactkv_amd.paged import PageTable, _popc16


def test_add_claims_full_and_open_pages():
    t = PageTable(num_pages=10, max_seqs=3, max_pages=4, device="cpu")
    assert t.add(0) == 0 and t.pages(0) == [0]                 # open page only
    assert t.add(16) == 1 and t.pages(1) == [1, 2]             # one full page + the open page
    assert t.add(64) == 2 and t.pages(2) == [3, 4, 5, 6]       # at capacity: no open page
    assert t.free_pages() == 3
    assert t.block_table[1, :2].tolist() == [1, 2] and t.lens.tolist() == [0, 16, 64]


def test_begin_step_opens_the_next_page_before_it_is_needed():
    t = PageTable(num_pages=8, max_seqs=2, max_pages=4, device="cpu")
    t.add(14)
    t.add(3)
    t.begin_step()
    assert t.length(0) == 15 and t.pages(0) == [0] and t.filled_in_step() == []
    t.begin_step([1, 0])                                       # slot 0's token 15 fills page 0
    assert t.pages(0) == [0, 2] and t.block_table[0, 1].item() == 2
    assert t.filled_in_step() == [(1, 0, 0)]                   # (row, slot, page index)
    slots, bt, lens = t.step_rows()
    assert slots.tolist() == [1, 0] and lens.tolist() == [5, 16] and bt[1, :2].tolist() == [0, 2]
    t.begin_step([0, 1])
    assert t.step_rows()[0] is None                            # dense rows: views, no gather


def test_release_returns_pages_and_failures_change_nothing():
    t = PageTable(num_pages=4, max_seqs=3, max_pages=4, device="cpu")
    a = t.add(30)
    b = t.add(15)
    assert t.free_pages() == 1
    t.begin_step()                                             # a: 31, b: 16 -> b opens a page
    assert t.free_pages() == 0
    with pytest.raises(RuntimeError, match="exhausted"):
        t.begin_step()                                         # a: 32 needs a page, none free
    assert t.length(a) == 31 and t.length(b) == 16             # nothing changed
    t.release(b)
    assert t.free_pages() == 2 and t.lens[b].item() == 0
    with pytest.raises(RuntimeError, match="begin_step"):
        t.step_rows()
    with pytest.raises(ValueError):
        t.begin_step([b])                                      # released slot
    t.begin_step([a])
    assert t.length(a) == 32 and len(t.pages(a)) == 3
    with pytest.raises(ValueError):
        t.add(5, slot=a)
    with pytest.raises(ValueError):
        t.add(65)


def test_full_sequence_stops():
    t = PageTable(num_pages=4, max_seqs=1, max_pages=2, device="cpu")
    t.add(31)
    t.begin_step()                                             # 32: fills the last page, opens none
    assert t.pages(0) == [0, 1]
    with pytest.raises(RuntimeError, match="full"):
        t.begin_step()


def test_popc16_matches_bin_count():
    x = torch.arange(1 << 16, dtype=torch.int32)
    want = torch.tensor([bin(i).count("1") for i in range(1 << 16)], dtype=torch.int32)
    assert torch.equal(_popc16(x), want)
