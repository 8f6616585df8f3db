"""GPU checks of the measurement aids behind `bench.py --ceilings` (fa_diag_mfma_ceiling,
fa_diag_stream_read; no counterpart in the reference). They run and return rates inside what
the part can do: positive and at most its spec (2.5 PFLOP/s dense bf16, 157.3 TFLOP/s f32
matrix, 8 TB/s HBM), with margin for clock and measurement error."""
import pytest

import flat_attention_amd as fa

pytestmark = pytest.mark.gpu


def test_mfma_ceiling_is_within_the_spec(hip):
    bf16 = hip.mfma_ceiling(False)
    assert 200.0 < bf16 < 2500.0 * 1.05
    f32 = hip.mfma_ceiling(True, fa.DTYPE_F32)
    assert 20.0 < f32 < 157.3 * 1.05


def test_stream_read_is_within_the_spec(hip):
    for depth in (4, 16):
        tbps = hip.stream_read(depth)
        assert 0.5 < tbps < 8.0 * 1.05, depth
    with pytest.raises(fa.FlatHipError):
        hip.stream_read(5)
