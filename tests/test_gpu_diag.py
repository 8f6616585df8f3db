"""GPU checks of the measurement aids behind `bench.py --ceilings` (libflat_diag.so:
fad_mfma_ceiling, fad_stream_read; no counterpart in the reference). They run and return rates
inside what the part can do: positive and at most its spec (2.5 PFLOP/s dense bf16, 157.3
TFLOP/s f32 matrix, 8 TB/s HBM), with margin for clock and measurement error."""
import pytest

from flat_attention_amd import diag

pytestmark = pytest.mark.gpu


def test_mfma_ceiling_is_within_the_spec():
    bf16 = diag.mfma_ceiling(0, False)
    assert 200.0 < bf16 < 2500.0 * 1.05
    f32 = diag.mfma_ceiling(0, True, diag.DTYPE_F32)
    assert 20.0 < f32 < 157.3 * 1.05


def test_stream_read_is_within_the_spec():
    for depth in (4, 16):
        tbps = diag.stream_read(0, depth)
        assert 0.5 < tbps < 8.0 * 1.05, depth
    with pytest.raises(diag.DiagError):
        diag.stream_read(0, 5)
