"""Host-side dispatch policy (no GPU): the row-count thresholds measured on MI355X."""
from ishizuki_amd import affine, ggml


def test_minimum_rows_is_two_at_every_size():
    # VerifyMatmul.minimumRows re-measured: one M-row verify call beats M GEMVs from M = 2
    for nbytes in (1_000, 1_638_400, 9_830_400, 27_852_800, 397_312_000):
        assert affine.minimum_rows(nbytes) == 2


def test_dense_from_rows():
    assert ggml.dense_from_rows(2_949_120) == 32
    assert ggml.dense_from_rows(73_728_000) == 48
    assert ggml.dense_from_rows(10_000_000) == 48
