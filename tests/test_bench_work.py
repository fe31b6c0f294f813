"""The bench's algorithmic work counts (CPU only): the trailing update's flops against
closed forms, and the batch plan the count reads against the chunking rule."""

import bench
from hi2_amd.hessian import BATCH_ELEMS, BLOCK_COLUMNS as L, ROW_ELEMS, _super_blocks, batch_rows


def _pairs(widths):
    """Flops of 2 R x rank x cols over every ordered block pair of one row: for blocks of
    the given widths spanning W columns, 2 sum_b w_b (columns after b) = W^2 - sum w_b^2."""
    w = sum(widths)
    return w * w - sum(x * x for x in widths)


def _widths(k):
    return [min(L, k - i) for i in range(0, k, L)]


def test_unfused_trailing_flops_is_every_cross_block_pair():
    cfg = bench.CFG3
    want = sum(n * _pairs(_widths(k)) for _, n, k, _ in cfg["linears"])
    assert bench.trailing_flops(cfg, fused_rows=0) == want


def test_fused_batches_drop_exactly_their_near_updates():
    cfg = bench.CFG3
    near = 0
    for inp in cfg["order"]:
        shapes = [(g, k, 0) for _, n, k, i in cfg["linears"] if i == inp
                  for g in bench.group_rows(n, cfg["alloc"])]
        for k, sizes, padded in batch_rows(shapes):
            if padded <= 8192:
                w = _widths(k)
                sb = _super_blocks(k)
                near += sum(sizes) * sum(_pairs(w[b:b + sb]) for b in range(0, len(w), sb))
    assert near > 0  # cfg3 has fused batches (o_proj's, down_proj's)
    assert bench.trailing_flops(cfg, fused_rows=8192) == bench.trailing_flops(cfg, 0) - near


def test_batch_plan_cuts_chunks_and_pads_multi_chunk_batches():
    k = 4096
    step = ROW_ELEMS // k
    plan = batch_rows([(step + 5, k, 0), (300, k, 0), (70, 14336, 0)])
    assert [(kk, s) for kk, s, _ in plan] == [(k, [step, 5, 300]), (14336, [70])]
    assert plan[0][2] == step + 128 + 384  # each chunk of a multi-chunk batch on 128 rows
    assert plan[1][2] == 70  # a lone chunk keeps its rows
    # a batch closes before it would pass BATCH_ELEMS weights
    per = BATCH_ELEMS // k
    plan = batch_rows([(step, k, 0)] * (per // step + 1))
    assert [sum(s) for _, s, _ in plan] == [per, step]
    assert bench.group_rows(4096, bench.CFG3["alloc"]) == [1229, 2867]
