"""Host block tables of the batched restore: shared full blocks are written
once under dedup, and a block shared while partial in some request forces
request-by-request restores."""
import numpy as np

from origami_amd.lossless.native_gpu import batch_block_tables


def test_disjoint_tables_unchanged():
    t, ok = batch_block_tables([[0, 1, 2], [3, 4]], [48, 32], 16, dedup=True)
    assert ok and [x.tolist() for x in t] == [[0, 1, 2], [3, 4]]


def test_shared_full_prefix_deduplicated_in_later_requests():
    tables = [[7, 8, 1, 2], [7, 8, 3], [7, 8, 9, 4, 5]]
    t, ok = batch_block_tables(tables, [64, 40, 80], 16, dedup=True)
    assert ok
    assert t[0].tolist() == [7, 8, 1, 2]
    assert t[1].tolist() == [-1, -1, 3]
    assert t[2].tolist() == [-1, -1, 9, 4, 5]


def test_shared_blocks_kept_without_dedup():
    tables = [[7, 8, 1], [7, 8, 3]]
    t, ok = batch_block_tables(tables, [48, 48], 16, dedup=False)
    assert ok and t[1].tolist() == [7, 8, 3]


def test_shared_partial_block_is_not_batchable():
    # block 8 is the partial last block of request 0 but full in request 1
    t, ok = batch_block_tables([[7, 8], [7, 8, 3]], [20, 48], 16, dedup=True)
    assert not ok
    assert t[1].tolist() == [7, 8, 3]  # untouched


def test_first_occurrence_may_be_in_any_order():
    t, ok = batch_block_tables([[5, 6], [6, 5], [5]], [32, 32, 16], 16, dedup=True)
    assert ok
    assert t[0].tolist() == [5, 6] and t[1].tolist() == [-1, -1] and t[2].tolist() == [-1]


def test_single_request_passes_through():
    t, ok = batch_block_tables([np.array([3, 3])], [32], 16, dedup=True)
    assert ok and t[0].tolist() == [3, 3]
