"""GPU parity of the padded variable-length projection prefill (M12,
ExternalVariableProjectionRotaryGroupedPipeline, src/wgpu_external_variable.rs).

Follows tests/wgpu_external_variable.rs: padded Q/K/V rows are poisoned (Q 1e20, K -1e20,
V 1e20) and must not influence any active row; every sequence's active rows match the oracle run
on that sequence alone (compact rows, its own origins); padded query rows are exactly O = 0 and
LSE = -inf. Numerics: f32 2e-5 + 1e-4|e|; bf16 2e-2.
"""
import numpy as np
import pytest

import oracle
from _inputs import bf16_round, f16_round, normal
from conftest import assert_close

import flat_attention_amd as fa

pytestmark = pytest.mark.gpu

F32_ATOL, F32_RTOL = 2e-5, 1e-4
H16_ATOL = 2e-2


def _fixture(n, phase):
    """Closed-form generator of tests/wgpu_external_variable.rs:55."""
    x = np.arange(n, dtype=np.float32) * np.float32(0.019) + np.float32(phase)
    return (np.sin(x) * np.float32(1.625) + np.cos(x * np.float32(0.37)) * np.float32(0.3125)).astype(np.float32)


def _run_case(hip, shape, meta, config, rotary, dtype, q, k, v, check_seqs=None):
    qw, kw = shape.q_heads * shape.head_dim, shape.kv_heads * shape.head_dim
    q, k, v = q.copy(), k.copy(), v.copy()
    for b, m in enumerate(meta):  # poison_padding :146
        q.reshape(shape.batch, shape.query_len, qw)[b, m.active_query_len:] = 1.0e20
        k.reshape(shape.batch, shape.kv_len, kw)[b, m.active_kv_len:] = -1.0e20
        v.reshape(shape.batch, shape.kv_len, kw)[b, m.active_kv_len:] = 1.0e20
    pipe = fa.HipVariableProjectionPipeline(hip, dtype)
    out = pipe.create_output_buffer(shape)
    bufs = [fa.DeviceBuffer.from_array(hip, fa.host_storage(x, dtype)) for x in (q, k, v)]
    lay = pipe.encode(bufs[0], bufs[1], bufs[2], out, shape, meta, config, rotary)
    res = fa.download_attention(out, lay, dtype)
    o = fa.storage_to_f32(res.output, dtype).reshape(shape.batch, shape.query_len, qw)
    lse = res.lse.reshape(shape.batch, shape.q_heads, shape.query_len)
    rnd = {fa.DTYPE_BF16: bf16_round, fa.DTYPE_F16: f16_round}.get(dtype, lambda x: x)
    for b, m in enumerate(meta):
        aq, ak = m.active_query_len, m.active_kv_len
        if check_seqs is None or b in check_seqs:
            q1 = rnd(q.reshape(shape.batch, shape.query_len, qw)[b, :aq].reshape(-1))
            k1 = rnd(k.reshape(shape.batch, shape.kv_len, kw)[b, :ak].reshape(-1))
            v1 = rnd(v.reshape(shape.batch, shape.kv_len, kw)[b, :ak].reshape(-1))
            eo, el = oracle.forward_projection_asymmetric(
                q1, k1, v1, 1, shape.q_heads, shape.kv_heads, aq, ak, shape.head_dim,
                m.query_position_offset, config.causal, rotary.theta,
                m.query_rope_position_offset, rotary.kv_position_offset, True,
                scale=config.softmax_scale)
            if dtype == fa.DTYPE_F32:
                assert_close(f"O[{b}]", o[b, :aq].reshape(-1), eo, F32_ATOL, F32_RTOL)
                assert_close(f"LSE[{b}]", lse[b, :, :aq].reshape(-1), el, F32_ATOL, F32_RTOL)
            else:
                assert_close(f"O[{b}]", o[b, :aq].reshape(-1), eo, H16_ATOL, 0.0)
                assert_close(f"LSE[{b}]", lse[b, :, :aq].reshape(-1), el, H16_ATOL, 0.0)
        assert np.all(o[b, aq:] == 0.0), f"padded O rows of sequence {b}"
        assert np.all(np.isneginf(lse[b, :, aq:])), f"padded LSE rows of sequence {b}"


# (f16: the poisoned padding overflows to inf on conversion, which is still never read)
@pytest.mark.filterwarnings("ignore:overflow encountered in cast")
@pytest.mark.parametrize("dtype", [fa.DTYPE_F32, fa.DTYPE_BF16, fa.DTYPE_F16])
def test_mixed_length_causal_gqa_matches_independent_oracles(hip, dtype):
    """tests/wgpu_external_variable.rs:295."""
    shape = fa.AsymmetricGroupedAttentionShape(2, 8, 2, 5, 9, 64, 0)
    meta = [fa.VariableLengthSequenceMetadata(3, 6, 3, 17),
            fa.VariableLengthSequenceMetadata(5, 9, 4, 29)]
    q = _fixture(shape.q_tensor_len(), 0.2)
    k = _fixture(shape.kv_tensor_len(), 0.8)
    v = _fixture(shape.kv_tensor_len(), 1.4)
    _run_case(hip, shape, meta, fa.FlatAttentionConfig(True),
              fa.VariableLengthRotaryEmbeddingConfig(10000.0, 11), dtype, q, k, v)


# (f16: the poisoned padding overflows to inf on conversion, which is still never read)
@pytest.mark.filterwarnings("ignore:overflow encountered in cast")
@pytest.mark.parametrize("dtype", [fa.DTYPE_F32, fa.DTYPE_BF16, fa.DTYPE_F16])
def test_mixed_length_noncausal_mqa_matches_independent_oracles(hip, dtype):
    """tests/wgpu_external_variable.rs:340 (head_dim 80, explicit scale 0.125, theta 5e5)."""
    shape = fa.AsymmetricGroupedAttentionShape(3, 8, 1, 6, 10, 80, 0)
    meta = [fa.VariableLengthSequenceMetadata(1, 4, 0, 7),
            fa.VariableLengthSequenceMetadata(4, 7, 0, 19),
            fa.VariableLengthSequenceMetadata(6, 10, 0, 31)]
    q = _fixture(shape.q_tensor_len(), 0.4)
    k = _fixture(shape.kv_tensor_len(), 1.0)
    v = _fixture(shape.kv_tensor_len(), 1.6)
    _run_case(hip, shape, meta, fa.FlatAttentionConfig(False, 0.125),
              fa.VariableLengthRotaryEmbeddingConfig(500000.0, 5), dtype, q, k, v)


def test_serving_sized_variable_batch_bf16(hip):
    """Four sequences of a padded serving batch (Hq32 Hkv8 D128, padded 700 query / 1500 K/V
    rows): chunks of different lengths appended after different cached prefixes, causal. Every
    sequence's padding is checked; two sequences' active rows against the oracle."""
    rng = np.random.default_rng(12)
    shape = fa.AsymmetricGroupedAttentionShape(4, 32, 8, 700, 1500, 128, 0)
    meta = []
    for aq, ak in ((700, 1500), (1, 1), (333, 1033), (64, 64)):
        meta.append(fa.VariableLengthSequenceMetadata(aq, ak, ak - aq, ak - aq + int(rng.integers(0, 50))))
    q = bf16_round(normal(shape.q_tensor_len(), 41))
    k = bf16_round(normal(shape.kv_tensor_len(), 42))
    v = bf16_round(normal(shape.kv_tensor_len(), 43))
    _run_case(hip, shape, meta, fa.FlatAttentionConfig(True),
              fa.VariableLengthRotaryEmbeddingConfig(10000.0, 0), fa.DTYPE_BF16, q, k, v,
              check_seqs=(1, 2))


def test_variable_pipeline_rejects_metadata_length_and_causal_overflow(hip):
    """tests/wgpu_external_variable.rs:390."""
    shape = fa.AsymmetricGroupedAttentionShape(1, 4, 2, 2, 4, 32, 0)
    pipe = fa.HipVariableProjectionPipeline(hip, fa.DTYPE_F32)
    q = fa.DeviceBuffer(hip, shape.q_tensor_len() * 4)
    kv = fa.DeviceBuffer(hip, shape.kv_tensor_len() * 4)
    out = pipe.create_output_buffer(shape)
    rot = fa.VariableLengthRotaryEmbeddingConfig(10000.0, 0)
    with pytest.raises(fa.FlatHipError) as e:
        pipe.encode(q, kv, kv, out, shape, [], fa.FlatAttentionConfig(), rot)
    assert e.value.variant == "LengthMismatch" and "active sequence metadata" in str(e.value)
    with pytest.raises(fa.FlatHipError) as e:
        pipe.encode(q, kv, kv, out, shape,
                    [fa.VariableLengthSequenceMetadata(1, 1, 2**32 - 1, 0)],
                    fa.FlatAttentionConfig(True), rot)
    assert e.value.variant == "PositionOverflow"
