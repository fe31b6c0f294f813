"""The GPTQ batch layout (CPU only): where a batch's working buffer pads its units."""

from hi2_amd.hessian import _padded


def test_runs_of_one_factor_are_unpadded_and_start_on_128_rows():
    a, b = object(), object()
    sizes = [37, 150, 70, 45, 29]
    got = _padded(sizes, [id(a), id(a), id(a), id(b), id(a)])
    assert got == [37, 150, 197, 128, 29]
    starts = [sum(got[:i]) for i in range(len(got))]
    assert starts[3] % 128 == 0 and starts[4] % 128 == 0  # each run on a 128-row boundary
    # the row classes of one input (the benchmark's down_proj): no padding at all
    assert _padded([1229, 2867], [1, 1]) == [1229, 2867]


def test_units_of_different_factors_each_start_on_128_rows():
    assert _padded([37, 150, 70, 29]) == [128, 256, 128, 29]
    assert _padded([300]) == [300]
    assert _padded([]) == []
