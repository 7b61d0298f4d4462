"""Host logic of the decode graph harness (no GPU): the captured batch sizes and
the size picked for a batch follow model_runner.py:264-269, 305."""
from nanovllm_amd.engine.decode_graphs import graph_batch_sizes, pick_graph_size


def test_graph_batch_sizes_match_reference():
    assert graph_batch_sizes(512) == [1, 2, 4, 8] + list(range(16, 513, 16))
    assert graph_batch_sizes(6) == [1, 2, 4]
    assert graph_batch_sizes(40) == [1, 2, 4, 8, 16, 32]


def test_pick_graph_size():
    gbs = graph_batch_sizes(512)
    assert pick_graph_size(gbs, 1) == 1
    assert pick_graph_size(gbs, 3) == 4
    assert pick_graph_size(gbs, 9) == 16
    assert pick_graph_size(gbs, 17) == 32
    assert pick_graph_size(gbs, 512) == 512
    assert pick_graph_size(gbs, 513) is None
