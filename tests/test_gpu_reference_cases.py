"""GPU mirrors of reference test cases on the asymmetric projection pass and the resident KV
cache, with each reference test's own shapes, deterministic fixtures and tolerances:
tests/m11_rectangular_wgpu.rs, tests/m14_resident_kv_cache.rs, tests/m15_external_resident.rs,
tests/m15_resident_decode.rs. Expected values come from the C oracle's asymmetric RoPE forward
(forward_reference_projection_grouped_rope_asymmetric, src/projection_asymmetric.rs:97)."""
import numpy as np
import pytest

import oracle
from conftest import assert_close

import flat_attention_amd as fa

pytestmark = pytest.mark.gpu


def _sin_fixture(n, phase):  # deterministic_values, tests/m11_rectangular_wgpu.rs:41
    i = np.arange(n, dtype=np.float32)
    return (np.sin(i * np.float32(0.137) + np.float32(phase)) * np.float32(0.6)).astype(np.float32)


def _mix_fixture(n, phase, step, a, freq, b):
    """x = i*step + phase; sin(x)*a + cos(x*freq)*b (the fixture of the M15/M48 tests)."""
    x = np.arange(n, dtype=np.float32) * np.float32(step) + np.float32(phase)
    return (np.sin(x) * np.float32(a) + np.cos(x * np.float32(freq)) * np.float32(b)).astype(
        np.float32)


def _buf(hip, x):
    return fa.DeviceBuffer.from_array(hip, np.ascontiguousarray(x, dtype=np.float32))


@pytest.mark.parametrize("query_len,kv_len,qpos,causal", [
    (3, 5, 0, False),  # rectangular_wgpu_matches_oracle_for_cross_attention :309
    (1, 7, 6, True),   # single_query_decode_matches_oracle_over_longer_kv :314
])
def test_m11_rectangular_matches_oracle(hip, query_len, kv_len, qpos, causal):
    """run_case tests/m11_rectangular_wgpu.rs:128: B1 Hq4 Hkv2 D8, Q rotated from qpos, raw K
    from 0; max |error| < 2e-4."""
    b, hq, hkv, D = 1, 4, 2, 8
    q = _sin_fixture(b * query_len * hq * D, 0.2)
    k = _sin_fixture(b * kv_len * hkv * D, 0.8)
    v = _sin_fixture(b * kv_len * hkv * D, 1.4)
    shape = fa.AsymmetricGroupedAttentionShape(b, hq, hkv, query_len, kv_len, D, qpos)
    rot = fa.AsymmetricRotaryEmbeddingConfig(1e4, qpos, 0)
    pipe = fa.HipAsymmetricProjectionPipeline(hip)
    out = pipe.create_output_buffer(shape)
    pipe.encode(_buf(hip, q), _buf(hip, k), _buf(hip, v), out, shape,
                fa.FlatAttentionConfig(causal), rot)
    res = fa.download_attention(out, pipe.layout(shape), fa.DTYPE_F32)
    eo, el = oracle.forward_projection_asymmetric(q, k, v, b, hq, hkv, query_len, kv_len, D, qpos,
                                                  causal, theta=1e4, q_rope_offset=qpos)
    assert np.max(np.abs(res.output - eo)) < 2e-4
    assert np.max(np.abs(res.lse - el)) < 2e-4


def test_m14_resident_append_preserves_prefix_and_batch_capacity_stride(hip):
    """resident_append_preserves_prefix_and_batch_capacity_stride
    tests/m14_resident_kv_cache.rs:102: batch 2, Hkv 2, capacity 5, D 4; two rows then one row
    land at cache row b * capacity + position, byte-exact, the prefix untouched."""
    batch, hkv, cap, D = 2, 2, 5, 4
    width = hkv * D
    cache = fa.HipResidentKvCache(hip, batch, hkv, cap, D)
    assert cache.is_empty() and cache.remaining_capacity() == cap
    first_k = 100.0 + np.arange(batch * 2 * width, dtype=np.float32)
    first_v = 500.0 + np.arange(batch * 2 * width, dtype=np.float32)
    assert cache.record_append(_buf(hip, first_k), _buf(hip, first_v), 2) == 2
    next_k = 900.0 + np.arange(batch * width, dtype=np.float32)
    next_v = 1300.0 + np.arange(batch * width, dtype=np.float32)
    assert cache.record_append(_buf(hip, next_k), _buf(hip, next_v), 1) == 3
    assert len(cache) == 3 and cache.remaining_capacity() == 2
    ak = cache.k_buffer().download(np.float32, batch * cap * width).reshape(batch, cap, width)
    av = cache.v_buffer().download(np.float32, batch * cap * width).reshape(batch, cap, width)
    fk, fv = first_k.reshape(batch, 2, width), first_v.reshape(batch, 2, width)
    for b in range(batch):
        assert np.array_equal(ak[b, :2], fk[b]) and np.array_equal(av[b, :2], fv[b])
        assert np.array_equal(ak[b, 2], next_k.reshape(batch, width)[b])
        assert np.array_equal(av[b, 2], next_v.reshape(batch, width)[b])


def test_m14_reset_reuses_prefix_without_copying_old_cache(hip):
    """reset_reuses_prefix_without_copying_old_cache tests/m14_resident_kv_cache.rs:183."""
    batch, hkv, cap, D = 2, 1, 4, 8
    width = hkv * D
    cache = fa.HipResidentKvCache(hip, batch, hkv, cap, D)
    init = np.full(batch * 2 * width, 3.0, np.float32)
    cache.record_append(_buf(hip, init), _buf(hip, init), 2)
    cache.reset()
    assert cache.is_empty()
    rk = 10.0 + np.arange(batch * width, dtype=np.float32)
    rv = 40.0 + np.arange(batch * width, dtype=np.float32)
    cache.record_append(_buf(hip, rk), _buf(hip, rv), 1)
    assert len(cache) == 1
    ak = cache.k_buffer().download(np.float32, batch * cap * width).reshape(batch, cap, width)
    av = cache.v_buffer().download(np.float32, batch * cap * width).reshape(batch, cap, width)
    for b in range(batch):
        assert np.array_equal(ak[b, 0], rk.reshape(batch, width)[b])
        assert np.array_equal(av[b, 0], rv.reshape(batch, width)[b])


def test_m14_append_rejects_capacity_overflow_and_short_sources(hip):
    """append_rejects_capacity_overflow_and_short_sources tests/m14_resident_kv_cache.rs:247."""
    cache = fa.HipResidentKvCache(hip, 1, 2, 2, 4)
    src = _buf(hip, np.ones(8, np.float32))
    cache.record_append(src, src, 1)
    with pytest.raises(fa.FlatHipError) as e:
        cache.record_append(src, src, 2)
    assert e.value.variant == "CapacityExceeded"
    assert "append 2 at length 1 exceeds capacity 2" in str(e.value)
    assert len(cache) == 1
    fresh = fa.HipResidentKvCache(hip, 2, 2, 4, 4)
    with pytest.raises(fa.FlatHipError) as e:
        fresh.record_append(src, src, 1)
    assert e.value.variant == "BufferTooSmall" and "K" in str(e.value)
    assert fresh.is_empty()


def _rotated_rows(raw, batch, kv_len, hkv, D, theta):
    return np.concatenate([oracle.rope_rotate_rows(raw.reshape(batch, -1)[b], kv_len, hkv, D,
                                                   theta) for b in range(batch)])


def test_m15_specialized_decode_consumes_external_capacity_strided_kv(hip):
    """specialized_decode_consumes_external_capacity_strided_kv_without_copy
    tests/m15_external_resident.rs:197: B2 Hq4 Hkv2 D32, 3 live rows in a capacity-7 layout
    whose dead rows hold 9999 / -8888 (never read); tolerance 2e-4 + 1e-3|e|."""
    batch, hq, hkv, kv_len, cap, D, theta = 2, 4, 2, 3, 7, 32, 1e4
    width = hkv * D
    fx = lambda n, ph: _mix_fixture(n, ph, 0.027, 1.3125, 0.31, 0.40625)  # noqa: E731
    q = fx(batch * hq * D, 0.2)
    raw_k = fx(batch * kv_len * width, 0.8)
    v = fx(batch * kv_len * width, 1.4)
    pk = np.full((batch, cap, width), 9999.0, np.float32)
    pv = np.full((batch, cap, width), -8888.0, np.float32)
    pk[:, :kv_len] = _rotated_rows(raw_k, batch, kv_len, hkv, D, theta).reshape(batch, kv_len, width)
    pv[:, :kv_len] = v.reshape(batch, kv_len, width)
    shape = fa.AsymmetricGroupedAttentionShape(batch, hq, hkv, 1, kv_len, D, kv_len - 1)
    pipe = fa.HipResidentDecodePipeline(hip)
    lay0 = pipe.layout(batch, hq, D)
    out = fa.DeviceBuffer(hip, lay0.combined_bytes)
    lay = pipe.encode_external_pre_rotated_k(
        _buf(hip, q), _buf(hip, pk), _buf(hip, pv), out, shape, fa.FlatAttentionConfig(True),
        fa.AsymmetricRotaryEmbeddingConfig(theta, kv_len - 1, 0), cap)
    assert lay.output_elements == batch * hq * D and lay.lse_elements == batch * hq
    res = fa.download_attention(out, lay, fa.DTYPE_F32)
    eo, el = oracle.forward_projection_asymmetric(q, raw_k, v, batch, hq, hkv, 1, kv_len, D,
                                                  kv_len - 1, True, theta=theta,
                                                  q_rope_offset=kv_len - 1)
    assert_close("O", res.output, eo, 2e-4, 1e-3)
    assert_close("LSE", res.lse, el, 2e-4, 1e-3)


def test_m15_external_decode_rejects_invalid_geometry_before_dispatch(hip):
    """external_decode_rejects_invalid_specialized_geometry_before_dispatch
    tests/m15_external_resident.rs:312 (query_len 2 is the reference's InvalidQueryLen, reported
    here as LengthMismatch)."""
    hq, hkv, D, kv_len, cap = 4, 2, 32, 3, 5
    q = _buf(hip, np.zeros(hq * D * 2, np.float32))
    kv = _buf(hip, np.zeros(cap * hkv * D, np.float32))
    out = fa.DeviceBuffer(hip, (2 * hq * D + 2 * hq) * 4)
    pipe = fa.HipResidentDecodePipeline(hip)
    cfg = fa.FlatAttentionConfig(True)
    rot = fa.AsymmetricRotaryEmbeddingConfig(1e4, kv_len - 1, 0)
    cases = [
        (fa.AsymmetricGroupedAttentionShape(1, hq, hkv, 2, kv_len, D, kv_len - 1), cap,
         "LengthMismatch"),
        (fa.AsymmetricGroupedAttentionShape(1, hq, hkv, 1, kv_len, D, 0), cap,
         "CausalVisibilityMismatch"),
        (fa.AsymmetricGroupedAttentionShape(1, hq, hkv, 1, kv_len, D, kv_len - 1), 2,
         "InvalidCacheLength"),
    ]
    for shape, capacity, variant in cases:
        with pytest.raises(fa.FlatHipError) as e:
            pipe.encode_external_pre_rotated_k(q, kv, kv, out, shape, cfg, rot, capacity)
        assert e.value.variant == variant, (shape, capacity)


def test_m15_resident_decode_matches_oracle_with_capacity_stride(hip):
    """resident_decode_matches_oracle_with_capacity_stride tests/m15_resident_decode.rs:178:
    B2 Hq4 Hkv2 D64, 5 rows appended (K pre-rotated) into a capacity-9 cache, decode at
    position 4; tolerance 2e-4 + 1e-3|e|."""
    batch, hq, hkv, kv_len, cap, D, theta = 2, 4, 2, 5, 9, 64, 1e4
    width = hkv * D
    fx = lambda n, ph: _mix_fixture(n, ph, 0.017, 1.25, 0.41, 0.375)  # noqa: E731
    q = fx(batch * hq * D, 0.15)
    raw_k = fx(batch * kv_len * width, 0.7)
    v = fx(batch * kv_len * width, 1.3)
    cache = fa.HipResidentKvCache(hip, batch, hkv, cap, D)
    cache.record_append(_buf(hip, _rotated_rows(raw_k, batch, kv_len, hkv, D, theta)),
                        _buf(hip, v), kv_len)
    pipe = fa.HipResidentDecodePipeline(hip)
    out = pipe.create_output_buffer(cache, hq)
    lay = pipe.encode(_buf(hip, q), cache, out, hq, fa.FlatAttentionConfig(True), theta,
                      kv_len - 1)
    res = fa.download_attention(out, lay, fa.DTYPE_F32)
    eo, el = oracle.forward_projection_asymmetric(q, raw_k, v, batch, hq, hkv, 1, kv_len, D,
                                                  kv_len - 1, True, theta=theta,
                                                  q_rope_offset=kv_len - 1)
    assert_close("O", res.output, eo, 2e-4, 1e-3)
    assert_close("LSE", res.lse, el, 2e-4, 1e-3)


# ---------------------------------------------------------------- grouped / rotary executors
def _fx(step, a, freq, b):
    return lambda n, ph: _mix_fixture(n, ph, step, a, freq, b)


GROUPED_SHAPES = [(1, 4, 4, 17, 32), (1, 8, 2, 17, 64), (2, 8, 1, 9, 80), (1, 16, 4, 5, 128)]


@pytest.mark.parametrize("dims", GROUPED_SHAPES)
@pytest.mark.parametrize("causal", [False, True])
def test_grouped_matches_oracle_for_mha_gqa_and_mqa(hip, dims, causal):
    """grouped_wgpu_matches_oracle_for_mha_gqa_and_mqa tests/wgpu_grouped.rs:47 (GQA without
    RoPE through the grouped executor), 6e-5 + 6e-4|e|."""
    b, hq, hkv, s, d = dims
    shape = fa.GroupedAttentionShape(b, hq, hkv, s, d)
    fx = _fx(0.021, 2.0, 0.73, 0.35)
    q, k, v = fx(shape.q_tensor_len(), 0.2), fx(shape.kv_tensor_len(), 0.9), fx(shape.kv_tensor_len(), 1.7)
    cfg = fa.FlatAttentionConfig(causal)
    got = fa.HipRotaryGroupedAttention(hip).forward(q, k, v, shape, cfg, None)
    eo, el = oracle.forward_grouped(q, k, v, b, hq, hkv, s, d, causal)
    assert_close("O", got.output, eo, 6e-5, 6e-4)
    assert_close("LSE", got.lse, el, 6e-5, 6e-4)


def test_resident_gqa_keeps_physical_kv_head_cardinality(hip):
    """resident_gqa_keeps_physical_kv_head_cardinality tests/wgpu_grouped.rs:101: K/V stay at
    Hkv = 3 heads (Q is 4x their size) and the resident result is one packed [O | LSE]."""
    b, hq, hkv, s, d = 2, 12, 3, 17, 64
    shape = fa.GroupedAttentionShape(b, hq, hkv, s, d)
    fx = _fx(0.021, 2.0, 0.73, 0.35)
    q, k, v = fx(shape.q_tensor_len(), 0.3), fx(shape.kv_tensor_len(), 1.1), fx(shape.kv_tensor_len(), 1.9)
    ex = fa.HipRotaryGroupedAttention(hip)
    bq, bk, bv = (ex.upload(x) for x in (q, k, v))
    assert bq.nbytes == 4 * bk.nbytes == 4 * bv.nbytes
    cfg = fa.FlatAttentionConfig(True)
    out = ex.forward_resident(bq, bk, bv, shape, cfg, None)
    lay = ex.layout(shape)
    assert lay.output_elements == shape.q_tensor_len() and lay.lse_elements == shape.lse_len()
    assert out.nbytes == lay.combined_bytes
    got = ex.download_attention(out, shape)
    eo, el = oracle.forward_grouped(q, k, v, b, hq, hkv, s, d, True)
    assert_close("O", got.output, eo, 6e-5, 6e-4)
    assert_close("LSE", got.lse, el, 6e-5, 6e-4)


def test_invalid_grouping_fails_before_dispatch(hip):
    """invalid_grouping_fails_before_dispatch tests/wgpu_grouped.rs:141."""
    shape = fa.GroupedAttentionShape(1, 6, 4, 2, 8)
    z = np.zeros(6 * 2 * 8, np.float32)
    with pytest.raises(fa.FlatHipError) as e:
        fa.HipRotaryGroupedAttention(hip).forward(z, z[:64], z[:64], shape,
                                                  fa.FlatAttentionConfig(), None)
    assert e.value.variant == "InvalidHeadGrouping"


@pytest.mark.parametrize("dims", GROUPED_SHAPES)
@pytest.mark.parametrize("theta,offset", [(1e4, 0), (5e5, 11)])
@pytest.mark.parametrize("causal", [False, True])
def test_fused_rope_grouped_matches_oracle(hip, dims, theta, offset, causal):
    """fused_rope_grouped_wgpu_matches_oracle tests/wgpu_rotary_grouped.rs:47, 1.5e-4 + 1e-3|e|."""
    b, hq, hkv, s, d = dims
    shape = fa.GroupedAttentionShape(b, hq, hkv, s, d)
    fx = _fx(0.017, 2.25, 0.43, 0.4)
    q, k, v = fx(shape.q_tensor_len(), 0.15), fx(shape.kv_tensor_len(), 0.85), fx(shape.kv_tensor_len(), 1.55)
    cfg = fa.FlatAttentionConfig(causal)
    got = fa.HipRotaryGroupedAttention(hip).forward(q, k, v, shape, cfg,
                                                    fa.RotaryEmbeddingConfig(theta, offset))
    eo, el = oracle.forward_grouped_rope(q, k, v, b, hq, hkv, s, d, causal, theta, offset)
    assert_close("O", got.output, eo, 1.5e-4, 1e-3)
    assert_close("LSE", got.lse, el, 1.5e-4, 1e-3)


def test_resident_rope_keeps_raw_qkv_cardinality_and_output_contract(hip):
    """resident_r1_keeps_raw_qkv_cardinality_and_no_rope_output_contract
    tests/wgpu_rotary_grouped.rs:112: B1 Hq12 Hkv3 S17 D64, scale 0.125, theta 1e4, offset 23;
    the caller's Q/K/V keep their raw cardinality and the output holds no rotated tensors."""
    b, hq, hkv, s, d = 1, 12, 3, 17, 64
    shape = fa.GroupedAttentionShape(b, hq, hkv, s, d)
    fx = _fx(0.017, 2.25, 0.43, 0.4)
    q, k, v = fx(shape.q_tensor_len(), 0.25), fx(shape.kv_tensor_len(), 0.95), fx(shape.kv_tensor_len(), 1.65)
    ex = fa.HipRotaryGroupedAttention(hip)
    bq, bk, bv = (ex.upload(x) for x in (q, k, v))
    assert bq.nbytes == 4 * bk.nbytes
    cfg = fa.FlatAttentionConfig(True, 0.125)
    rot = fa.RotaryEmbeddingConfig(1e4, 23)
    out = ex.forward_resident(bq, bk, bv, shape, cfg, rot)
    assert out.nbytes == (shape.q_tensor_len() + shape.lse_len()) * 4
    assert np.array_equal(bk.download(np.float32, k.size), k)  # inputs are not rotated in place
    got = ex.download_attention(out, shape)
    eo, el = oracle.forward_grouped_rope(q, k, v, b, hq, hkv, s, d, True, 1e4, 23, scale=0.125)
    assert_close("O", got.output, eo, 1.5e-4, 1e-3)
    assert_close("LSE", got.lse, el, 1.5e-4, 1e-3)


# ----------------------------------------------------------- caller-owned projection passes
def _proj_oracle(q, k, v, shape, causal, theta, offset):
    return oracle.forward_projection_asymmetric(
        q, k, v, shape.batch, shape.q_heads, shape.kv_heads, shape.seq_len, shape.seq_len,
        shape.head_dim, 0, causal, theta=theta, q_rope_offset=offset, kv_rope_offset=offset)


def test_caller_can_encode_two_flat_passes_then_submit_once(hip):
    """caller_can_encode_two_flat_passes_then_submit_once tests/wgpu_external.rs:135: a causal
    and a full pass over the same buffers are enqueued back to back on the library's stream and
    read once; 1.5e-4 + 1e-3|e|."""
    shape = fa.GroupedAttentionShape(1, 8, 2, 17, 64)
    fx = _fx(0.019, 2.125, 0.47, 0.34375)
    q, k, v = fx(shape.q_tensor_len(), 0.2), fx(shape.kv_tensor_len(), 0.8), fx(shape.kv_tensor_len(), 1.4)
    rot = fa.RotaryEmbeddingConfig(1e4, 13)
    pipe = fa.HipProjectionRotaryGroupedPipeline(hip)
    bq, bk, bv = _buf(hip, q), _buf(hip, k), _buf(hip, v)
    oc, of = pipe.create_output_buffer(shape), pipe.create_output_buffer(shape)
    lay_c = pipe.encode(bq, bk, bv, oc, shape, fa.FlatAttentionConfig(True), rot)
    lay_f = pipe.encode(bq, bk, bv, of, shape, fa.FlatAttentionConfig(False), rot)
    hip.synchronize()
    for out, lay, causal in ((oc, lay_c, True), (of, lay_f, False)):
        got = fa.download_attention(out, lay, fa.DTYPE_F32)
        eo, el = _proj_oracle(q, k, v, shape, causal, 1e4, 13)
        assert_close(f"O causal={causal}", got.output, eo, 1.5e-4, 1e-3)
        assert_close(f"LSE causal={causal}", got.lse, el, 1.5e-4, 1e-3)


def test_external_pipeline_handles_mqa_and_rejects_short_buffers(hip):
    """external_pipeline_handles_mqa_and_rejects_short_buffers tests/wgpu_external.rs:250:
    B2 Hq8 Hkv1 S9 D80, theta 5e5, offset 21, causal; a 4-byte Q is BufferTooSmall."""
    shape = fa.GroupedAttentionShape(2, 8, 1, 9, 80)
    fx = _fx(0.019, 2.125, 0.47, 0.34375)
    q, k, v = fx(shape.q_tensor_len(), 0.2), fx(shape.kv_tensor_len(), 0.8), fx(shape.kv_tensor_len(), 1.4)
    rot = fa.RotaryEmbeddingConfig(5e5, 21)
    pipe = fa.HipProjectionRotaryGroupedPipeline(hip)
    out = pipe.create_output_buffer(shape)
    bk, bv = _buf(hip, k), _buf(hip, v)
    lay = pipe.encode(_buf(hip, q), bk, bv, out, shape, fa.FlatAttentionConfig(True), rot)
    got = fa.download_attention(out, lay, fa.DTYPE_F32)
    eo, el = _proj_oracle(q, k, v, shape, True, 5e5, 21)
    assert_close("O", got.output, eo, 1.5e-4, 1e-3)
    assert_close("LSE", got.lse, el, 1.5e-4, 1e-3)
    with pytest.raises(fa.FlatHipError) as e:
        pipe.encode(fa.DeviceBuffer(hip, 4), bk, bv, out, shape, fa.FlatAttentionConfig(True), rot)
    assert e.value.variant == "BufferTooSmall" and "Q" in str(e.value)


@pytest.mark.parametrize("case", [
    # single_query_decode_reads_long_resident_gqa_cache tests/wgpu_external_asymmetric.rs:199
    ((1, 8, 2, 1, 17, 64, 16), True, (1e4, 29, 13), 0.2),
    # rectangular_noncausal_mqa_matches_oracle :231
    ((2, 8, 1, 5, 9, 80, 0), False, (5e5, 3, 101), 0.4),
    # vec4_gqa_prefill_matches_oracle_for_product_shapes :262 (no vector variant here: one kernel)
    ((1, 8, 2, 17, 17, 64, 0), False, (1e4, 0, 0), 0.7 + 64 * 0.001),
    ((1, 8, 2, 17, 17, 64, 0), True, (1e4, 0, 0), 0.7 + 64 * 0.001),
    ((1, 8, 2, 17, 17, 128, 0), False, (1e4, 0, 0), 0.7 + 128 * 0.001),
    ((1, 8, 2, 17, 17, 128, 0), True, (1e4, 0, 0), 0.7 + 128 * 0.001),
])
def test_external_asymmetric_cases_match_oracle(hip, case):
    """run_case tests/wgpu_external_asymmetric.rs:135: raw K rotated in the kernel, RoPE offsets
    apart from the causal offset; 1.5e-4 + 1e-3|e|."""
    dims, causal, (theta, qro, kro), phase = case
    b, hq, hkv, ql, kl, d, qpos = dims
    shape = fa.AsymmetricGroupedAttentionShape(*dims)
    fx = _fx(0.023, 1.875, 0.41, 0.28125)
    q = fx(shape.q_tensor_len(), phase)
    k = fx(b * kl * hkv * d, phase + 0.6)
    v = fx(b * kl * hkv * d, phase + 1.2)
    pipe = fa.HipAsymmetricProjectionPipeline(hip)
    out = pipe.create_output_buffer(shape)
    pipe.encode(_buf(hip, q), _buf(hip, k), _buf(hip, v), out, shape,
                fa.FlatAttentionConfig(causal), fa.AsymmetricRotaryEmbeddingConfig(theta, qro, kro))
    got = fa.download_attention(out, pipe.layout(shape), fa.DTYPE_F32)
    eo, el = oracle.forward_projection_asymmetric(q, k, v, b, hq, hkv, ql, kl, d, qpos, causal,
                                                  theta=theta, q_rope_offset=qro,
                                                  kv_rope_offset=kro)
    assert_close("O", got.output, eo, 1.5e-4, 1e-3)
    assert_close("LSE", got.lse, el, 1.5e-4, 1e-3)


def test_rectangular_pipeline_rejects_short_kv_buffer(hip):
    """rectangular_pipeline_rejects_short_kv_buffer tests/wgpu_external_asymmetric.rs:324."""
    shape = fa.AsymmetricGroupedAttentionShape(1, 4, 2, 1, 8, 32, 7)
    fx = _fx(0.023, 1.875, 0.41, 0.28125)
    pipe = fa.HipAsymmetricProjectionPipeline(hip)
    kv = _buf(hip, fx(8 * 2 * 32, 0.9))
    with pytest.raises(fa.FlatHipError) as e:
        pipe.encode(_buf(hip, fx(4 * 32, 0.3)), fa.DeviceBuffer(hip, 4), kv,
                    pipe.create_output_buffer(shape), shape, fa.FlatAttentionConfig(True),
                    fa.AsymmetricRotaryEmbeddingConfig(1e4, 7, 0))
    assert e.value.variant == "BufferTooSmall" and "K" in str(e.value)


@pytest.mark.parametrize("hq,hkv,kv_len,D,theta", [
    (8, 2, 17, 64, 1e4),   # prerotated_k_gqa_decode_matches_raw_k_m11_oracle :227
    (8, 1, 65, 80, 5e5),   # prerotated_k_mqa_decode_crosses_tile_boundary :232
])
def test_prerotated_k_decode_matches_raw_k_oracle(hip, hq, hkv, kv_len, D, theta):
    """run_decode_case tests/wgpu_prerotated_k_decode.rs:157: encode_pre_rotated_k at
    query_len 1, query position kv_len - 1, K rotated on the host; 1.5e-4 + 1e-3|e|."""
    pos = kv_len - 1
    shape = fa.AsymmetricGroupedAttentionShape(1, hq, hkv, 1, kv_len, D, pos)
    fx = _fx(0.021, 1.75, 0.43, 0.34375)
    q = fx(hq * D, 0.2)
    raw_k = fx(kv_len * hkv * D, 0.8)
    v = fx(kv_len * hkv * D, 1.4)
    k = oracle.rope_rotate_rows(raw_k, kv_len, hkv, D, theta)
    pipe = fa.HipAsymmetricProjectionPipeline(hip)
    out = pipe.create_output_buffer(shape)
    pipe.encode_pre_rotated_k(_buf(hip, q), _buf(hip, k), _buf(hip, v), out, shape,
                              fa.FlatAttentionConfig(True),
                              fa.AsymmetricRotaryEmbeddingConfig(theta, pos, 0))
    got = fa.download_attention(out, pipe.layout(shape), fa.DTYPE_F32)
    eo, el = oracle.forward_projection_asymmetric(q, raw_k, v, 1, hq, hkv, 1, kv_len, D, pos,
                                                  True, theta=theta, q_rope_offset=pos)
    assert_close("O", got.output, eo, 1.5e-4, 1e-3)
    assert_close("LSE", got.lse, el, 1.5e-4, 1e-3)


# ----------------------------------------------------------------------- chunked prefill
@pytest.mark.parametrize("dims,causal,chunk", [((2, 4, 2, 7, 32), True, 3),
                                               ((2, 4, 1, 5, 32), False, 2)])
def test_m16_chunked_prefill_matches_contiguous_oracle(hip, dims, causal, chunk):
    """chunked_prefill_matches_contiguous_oracle_for_gqa_and_mqa
    tests/m16_chunked_prefill_wgpu.rs:217 (theta 1e4, offset 5), 2e-4 + 1e-3|e|, against both the
    chunked and the contiguous oracle."""
    b, hq, hkv, s, d = dims
    shape = fa.GroupedAttentionShape(*dims)
    fx = _fx(0.019, 1.1875, 0.37, 0.34375)
    q, k, v = fx(shape.q_tensor_len(), 0.2), fx(shape.kv_tensor_len(), 0.8), fx(shape.kv_tensor_len(), 1.4)
    pipe = fa.HipChunkedProjectionPrefillPipeline(hip)
    out = fa.DeviceBuffer(hip, fa.packed_layout(q.size, shape.lse_len(), fa.DTYPE_F32).combined_bytes)
    pipe.encode(_buf(hip, q), _buf(hip, k), _buf(hip, v), out, shape,
                fa.FlatAttentionConfig(causal), fa.RotaryEmbeddingConfig(1e4, 5), chunk)
    got = fa.download_attention(out, fa.packed_layout(q.size, shape.lse_len(), fa.DTYPE_F32),
                                fa.DTYPE_F32)
    eo, el = oracle.chunked_prefill(q, k, v, b, hq, hkv, s, d, causal, 1e4, 5, chunk)
    assert_close("O", got.output, eo, 2e-4, 1e-3)
    assert_close("LSE", got.lse, el, 2e-4, 1e-3)
    co, cl = _proj_oracle(q, k, v, shape, causal, 1e4, 5)
    assert_close("O (contiguous)", got.output, co, 2e-4, 1e-3)
    assert_close("LSE (contiguous)", got.lse, cl, 2e-4, 1e-3)


def test_m16_zero_chunk_is_rejected_before_recording(hip):
    """zero_chunk_is_rejected_before_recording tests/m16_chunked_prefill_wgpu.rs:249."""
    shape = fa.GroupedAttentionShape(1, 2, 1, 2, 8)
    fx = _fx(0.019, 1.1875, 0.37, 0.34375)
    bq, bkv = _buf(hip, fx(32, 0.1)), _buf(hip, fx(16, 0.5))
    out = fa.DeviceBuffer(hip, 1024)
    with pytest.raises(fa.FlatHipError) as e:
        fa.HipChunkedProjectionPrefillPipeline(hip).encode(
            bq, bkv, bkv, out, shape, fa.FlatAttentionConfig(True),
            fa.RotaryEmbeddingConfig(1e4, 0), 0)
    assert e.value.variant == "ZeroQueryChunkSize"


# ------------------------------------------------------------ public forward reuse, chain
def test_m25_grouped_forward_pipeline_reuses_across_gqa_and_mqa(hip):
    """public_grouped_forward_pipeline_reuses_across_gqa_and_mqa
    tests/m25_wgpu_public_forward_reuse.rs:198: one executor, three encodes into the same output
    per case, GQA (1,4,2,7,16) causal and MQA (2,4,1,5,8) with scale 0.31; 6e-4 + 2.5e-3|e|."""
    ex = fa.HipRotaryGroupedAttention(hip)
    fx = _fx(0.043, 0.7, 0.37, 0.3)
    for dims, cfg, phase in (((1, 4, 2, 7, 16), fa.FlatAttentionConfig(True), 0.1),
                             ((2, 4, 1, 5, 8), fa.FlatAttentionConfig(False, 0.31), 1.7)):
        b, hq, hkv, s, d = dims
        shape = fa.GroupedAttentionShape(*dims)
        q = fx(shape.q_tensor_len(), phase)
        k, v = fx(shape.kv_tensor_len(), phase + 0.6), fx(shape.kv_tensor_len(), phase + 1.2)
        eo, el = oracle.forward_grouped(q, k, v, b, hq, hkv, s, d, cfg.causal, scale=cfg.softmax_scale)
        bq, bk, bv = (ex.upload(x) for x in (q, k, v))
        out = fa.DeviceBuffer(hip, ex.layout(shape).combined_bytes)
        for reuse in range(3):
            ex.forward_resident(bq, bk, bv, shape, cfg, None, out)
            got = ex.download_attention(out, shape)
            assert_close(f"reuse {reuse} O", got.output, eo, 6e-4, 2.5e-3)
            assert_close(f"reuse {reuse} LSE", got.lse, el, 6e-4, 2.5e-3)


@pytest.mark.parametrize("dims,cfg", [((1, 4, 2, 7, 16), (True, None)),
                                      ((2, 4, 1, 5, 8), (False, 0.31))])
def test_m26_resident_training_chain_matches_oracle(hip, dims, cfg):
    """public_resident_{gqa,mqa}_training_chain_matches_oracle
    tests/m26_wgpu_public_training_chain.rs:318,335: resident forward, its O and LSE packed with
    Q, K, V, dO into the backward's Q|K|V|dO|O|LSE contract, one backward; forward and
    gradients against the oracles; 6e-4 + 2.5e-3|e|."""
    b, hq, hkv, s, d = dims
    shape = fa.GroupedAttentionShape(*dims)
    config = fa.FlatAttentionConfig(*cfg)
    fx = _fx(0.043, 0.7, 0.37, 0.3)
    q, k, v = fx(shape.q_tensor_len(), 0.1), fx(shape.kv_tensor_len(), 0.7), fx(shape.kv_tensor_len(), 1.3)
    do = fx(shape.q_tensor_len(), 1.9)
    eo, el = oracle.forward_grouped(q, k, v, b, hq, hkv, s, d, config.causal,
                                    scale=config.softmax_scale)
    edq, edk, edv = oracle.backward_grouped(q, k, v, do, eo, el, b, hq, hkv, s, d, config.causal,
                                            scale=config.softmax_scale)
    ex = fa.HipRotaryGroupedAttention(hip)
    out = ex.forward_resident(ex.upload(q), ex.upload(k), ex.upload(v), shape, config, None)
    fwd = ex.download_attention(out, shape)
    assert_close("O", fwd.output, eo, 6e-4, 2.5e-3)
    assert_close("LSE", fwd.lse, el, 6e-4, 2.5e-3)
    pipe = fa.HipGroupedBackwardRecomputePipeline(hip)
    packed = fa.DeviceBuffer.from_array(
        hip, fa.pack_grouped_backward_recompute_inputs(q, k, v, do, fwd, shape))
    grads = pipe.create_gradient_buffer(shape)
    lay = pipe.encode(packed, grads, shape, config)
    g = grads.download(np.float32, lay.gradient_bytes // 4)  # offsets are in bytes
    dq = g[lay.dq_offset // 4:][:lay.q_elements]
    dk = g[lay.dk_offset // 4:][:lay.kv_elements]
    dv = g[lay.dv_offset // 4:][:lay.kv_elements]
    for name, a, e in (("dQ", dq, edq), ("dK", dk, edk), ("dV", dv, edv)):
        assert_close(name, a, e, 6e-4, 2.5e-3)


# ------------------------------------------------------------------ MHA executor matrix
def _matrix_fixture(shape, phase):  # tests/wgpu_matrix.rs:24
    i = np.arange(shape.tensor_len(), dtype=np.float32)
    ph = np.float32(phase)
    q = (np.sin(i * np.float32(0.037) + ph) * np.float32(0.85)).astype(np.float32)
    k = (np.cos(i * np.float32(0.053) - ph * np.float32(0.7)) * np.float32(0.72)).astype(np.float32)
    v = (np.sin(i * np.float32(0.029) + ph * np.float32(1.3)) * np.float32(1.15)).astype(np.float32)
    return q, k, v


def _check_mha(hip, shape, causal, phase, scale=None, qkv=None):
    """check_case tests/wgpu_matrix.rs:50: 5e-5 + 5e-4|e|."""
    q, k, v = qkv if qkv is not None else _matrix_fixture(shape, phase)
    cfg = fa.FlatAttentionConfig(causal, scale)
    got = fa.HipFlatAttention(hip).forward(q, k, v, shape, cfg)
    assert np.all(np.isfinite(got.output)) and np.all(np.isfinite(got.lse))
    eo, el = oracle.forward(q, k, v, shape.batch, shape.heads, shape.seq_len, shape.head_dim,
                            causal, scale=scale)
    assert_close("O", got.output, eo, 5e-5, 5e-4)
    assert_close("LSE", got.lse, el, 5e-5, 5e-4)


@pytest.mark.parametrize("case,head_dim", list(enumerate([1, 8, 16, 32, 64, 80, 96, 128])))
def test_every_supported_head_dimension_matches_reference(hip, case, head_dim):
    """every_supported_head_dimension_matches_reference tests/wgpu_matrix.rs:62."""
    shape = fa.AttentionShape(1, 2, 9, head_dim)
    _check_mha(hip, shape, False, 0.11 + case * 0.07)
    _check_mha(hip, shape, True, 0.19 + case * 0.05)


def test_sequence_tile_boundaries_match_reference(hip):
    """sequence_tile_boundaries_match_reference tests/wgpu_matrix.rs:79."""
    for case, s in enumerate([1, 7, 8, 9, 15, 16, 17, 31, 32, 63, 64, 65, 127, 128, 129]):
        _check_mha(hip, fa.AttentionShape(1, 1, s, 16), case % 2 == 0, 0.23 + case * 0.031)


def test_multiple_batches_and_heads_match_reference(hip):
    """multiple_batches_and_heads_match_reference tests/wgpu_matrix.rs:104."""
    shape = fa.AttentionShape(3, 4, 17, 32)
    _check_mha(hip, shape, False, 0.41)
    _check_mha(hip, shape, True, 0.67)


def test_high_dynamic_range_scores_remain_finite_and_match_reference(hip):
    """high_dynamic_range_scores_remain_finite_and_match_reference tests/wgpu_matrix.rs:119:
    +-8 queries against +-7 / +-6.5 keys at scale 0.125."""
    shape = fa.AttentionShape(1, 2, 17, 32)
    i = np.arange(shape.tensor_len())
    q = np.where(i % 2 == 0, 8.0, -8.0).astype(np.float32)
    k = np.array([7.0, -7.0, -6.5, 6.5], np.float32)[i % 4]
    v = (np.sin(i.astype(np.float32) * np.float32(0.017) - np.float32(0.3)) * 3.0).astype(np.float32)
    for causal in (False, True):
        _check_mha(hip, shape, causal, 0.0, scale=0.125, qkv=(q, k, v))


def test_causal_first_query_uses_only_first_value_row(hip):
    """causal_first_query_uses_only_first_value_row tests/wgpu_matrix.rs:161: exact equality."""
    shape = fa.AttentionShape(1, 1, 9, 8)
    z = np.zeros(shape.tensor_len(), np.float32)
    v = (np.arange(9, dtype=np.float32)[:, None] * 1000.0
         + np.arange(8, dtype=np.float32)[None, :]).reshape(-1)
    got = fa.HipFlatAttention(hip).forward(z, z, v, shape, fa.FlatAttentionConfig(True))
    assert np.array_equal(got.output[:8], v[:8])


def test_excessive_head_dimension_is_rejected_before_dispatch(hip):
    """excessive_head_dimension_is_rejected_before_dispatch tests/wgpu_matrix.rs:200."""
    shape = fa.AttentionShape(1, 1, 2, 129)
    z = np.zeros(shape.tensor_len(), np.float32)
    with pytest.raises(fa.FlatHipError) as e:
        fa.HipFlatAttention(hip).forward(z, z, z, shape, fa.FlatAttentionConfig())
    assert e.value.variant == "UnsupportedHeadDim"
    assert "129" in str(e.value) and "128" in str(e.value)


# ------------------------------------------------------------------ passive telemetry (M29)
def _same_dispatch(snap, real):
    for f in ("kernel_id", "kernel_name", "query_rows", "kv_rows", "workgroups", "workgroup_size",
              "dispatch_count", "temporary_allocation_count", "temporary_allocation_bytes",
              "splits", "fallback_reason", "device_name", "device_arch", "device_fingerprint"):
        assert getattr(snap, f) == getattr(real, f), (f, getattr(snap, f), getattr(real, f))


@pytest.mark.parametrize("case", [
    ("mha", (1, 4, 9, 32), fa.DTYPE_F32, None, {}),
    ("mha", (2, 2, 300, 128), fa.DTYPE_BF16, None, {}),
    ("gqa", (2, 8, 2, 130, 128), fa.DTYPE_BF16, (1e4, 3), {}),
    ("gqa", (1, 6, 1, 77, 64), fa.DTYPE_F16, (5e5, 0), {"precision": 1}),
    ("gqa", (1, 8, 2, 65, 128), fa.DTYPE_BF16, (1e4, 0), {"kernel": 0}),
    ("gqa", (1, 4, 2, 33, 6), fa.DTYPE_F32, (1e4, 0), {}),
    ("gqa", (1, 4, 2, 33, 64), fa.DTYPE_F32, (1e4, 0), {"prerotate": 0}),
])
def test_passive_telemetry_snapshot_matches_the_dispatch(case):
    """passive_snapshot_matches_selected_portable_dispatch tests/m29_runtime_telemetry.rs:7: the
    snapshot names the kernel, geometry, dispatch count and fallback reason the forward then
    reports for a resident forward, and submits nothing (the last dispatch's record is
    unchanged by it). A fresh
    context is used so the predicted allocations (RoPE table, workspaces) are the first call's;
    a second snapshot after the call predicts none."""
    kind, dims, dtype, rope, pol = case
    ctx = fa.HipContext(0)
    try:
        if "precision" in pol:
            ctx.set_prefill_precision(pol["precision"])
        if "kernel" in pol:
            ctx.set_prefill_kernel(pol["kernel"])
        if "prerotate" in pol:
            ctx.set_prefill_policy(pol["prerotate"])
        cfg = fa.FlatAttentionConfig(True)
        rng = np.random.default_rng(7)
        if kind == "mha":
            shape = fa.AttentionShape(*dims)
            ex = fa.HipFlatAttention(ctx, dtype)
            snap = ex.runtime_telemetry(shape, cfg)
            assert ctx.last_telemetry().kernel_id == "None"
            x = [ex.upload(rng.standard_normal(shape.tensor_len()).astype(np.float32))
                 for _ in range(3)]
            ex.forward_resident(*x, shape, cfg)
        else:
            shape = fa.GroupedAttentionShape(*dims)
            rot = fa.RotaryEmbeddingConfig(*rope) if rope else None
            ex = fa.HipRotaryGroupedAttention(ctx, dtype)
            snap = ex.runtime_telemetry(shape, cfg, rot)
            assert ctx.last_telemetry().kernel_id == "None"
            q = rng.standard_normal(shape.q_tensor_len()).astype(np.float32)
            k, v = (rng.standard_normal(shape.kv_tensor_len()).astype(np.float32) for _ in range(2))
            bq, bk, bv = (ex.upload(t) for t in (q, k, v))
            ex.forward_resident(bq, bk, bv, shape, cfg, rot)
        real = ctx.last_telemetry()
        _same_dispatch(snap, real)
        assert real.device_name and real.device_arch.startswith("gfx950")  # m29 :33-34
        if kind == "gqa" and rope and dims[-1] % 8 and dtype == fa.DTYPE_F32:
            assert real.fallback_reason == ("K pre-rotation pass needs head_dim % 8 == 0; "
                                            "K rotated on load")
        again = (ex.runtime_telemetry(shape, cfg) if kind == "mha"
                 else ex.runtime_telemetry(shape, cfg, rot))
        assert again.temporary_allocation_count == 0 and again.temporary_allocation_bytes == 0
        assert ctx.last_telemetry() == real
    finally:
        ctx.close()


# ------------------------------------------------------- repeatability (numerical policy)
def _policy_fixture(shape):  # tests/wgpu_numerical_policy.rs:20
    i = np.arange(shape.tensor_len())
    fi = i.astype(np.float32)
    q = (np.where(i % 3 == 0, -1.0, 1.0).astype(np.float32)
         * (np.sin(fi * np.float32(0.027)) * np.float32(3.5) + np.float32(0.125))).astype(np.float32)
    k = (np.where((i // 5) % 2 == 0, 1.0, -1.0).astype(np.float32)
         * (np.cos(fi * np.float32(0.019)) * np.float32(2.75) - np.float32(0.0625))).astype(np.float32)
    v = (np.sin(fi * np.float32(0.013)) * np.float32(4.0)).astype(np.float32)
    return q, k, v


@pytest.mark.parametrize("seq_len,head_dim", [(17, 64), (33, 80), (9, 128)])
@pytest.mark.parametrize("causal", [False, True])
def test_forward_is_bit_repeatable_on_same_context(hip, seq_len, head_dim, causal):
    """deterministic_mode_is_bit_repeatable_on_same_context tests/wgpu_numerical_policy.rs:84:
    every kernel here has one writer per output element and a fixed reduction order, so repeated
    forwards give the same bits; the first matches the oracle to 5e-5 + 5e-4|e|."""
    shape = fa.AttentionShape(1, 2, seq_len, head_dim)
    q, k, v = _policy_fixture(shape)
    cfg = fa.FlatAttentionConfig(causal, 0.125)
    ex = fa.HipFlatAttention(hip)
    first = ex.forward(q, k, v, shape, cfg)
    for it in range(4):
        again = ex.forward(q, k, v, shape, cfg)
        assert np.array_equal(again.output.view(np.uint32), first.output.view(np.uint32)), it
        assert np.array_equal(again.lse.view(np.uint32), first.lse.view(np.uint32)), it
    eo, el = oracle.forward(q, k, v, 1, 2, seq_len, head_dim, causal, scale=0.125)
    assert_close("O", first.output, eo, 5e-5, 5e-4)
    assert_close("LSE", first.lse, el, 5e-5, 5e-4)


def test_host_input_validation_names_the_non_finite_element(hip):
    """deterministic_mode_preserves_host_input_validation tests/wgpu_numerical_policy.rs:162:
    a NaN at Q[7] is NonFiniteInput naming Q and index 7."""
    shape = fa.AttentionShape(1, 1, 1, 64)
    q = np.zeros(64, np.float32)
    q[7] = np.nan
    z = np.zeros(64, np.float32)
    with pytest.raises(fa.FlatHipError) as e:
        fa.HipFlatAttention(hip).forward(q, z, z, shape, fa.FlatAttentionConfig())
    assert e.value.variant == "NonFiniteInput"
    assert "Q" in str(e.value) and "7" in str(e.value)


# --------------------------------------------------------------- M3 device matrix (MHA)
def _m3_fixture(shape):  # tests/wgpu_device.rs:12
    i = np.arange(shape.tensor_len(), dtype=np.float32)
    q = (np.sin(i * np.float32(0.071) - np.float32(0.8)) * np.float32(0.75)).astype(np.float32)
    k = (np.cos(i * np.float32(0.113) + np.float32(0.2)) * np.float32(0.65)).astype(np.float32)
    v = (np.sin(i * np.float32(0.047) - np.float32(0.4)) * np.float32(1.25)).astype(np.float32)
    return q, k, v


def _m3_parity(hip, shape, causal, qkv=None, scale=None, tol=((2e-5, 2e-4), (3e-5, 3e-4))):
    """assert_forward_parity tests/wgpu_device.rs:64: O 2e-5 + 2e-4|e|, LSE 3e-5 + 3e-4|e|."""
    q, k, v = qkv if qkv is not None else _m3_fixture(shape)
    got = fa.HipFlatAttention(hip).forward(q, k, v, shape, fa.FlatAttentionConfig(causal, scale))
    eo, el = oracle.forward(q, k, v, shape.batch, shape.heads, shape.seq_len, shape.head_dim,
                            causal, scale=scale)
    assert_close("O", got.output, eo, *tol[0])
    assert_close("LSE", got.lse, el, *tol[1])


def test_m3_head_dimension_matrix_matches_reference(hip):
    """m3_head_dimension_matrix_matches_reference tests/wgpu_device.rs:96."""
    for d in [1, 8, 16, 32, 64, 80, 96, 128]:
        for causal in (False, True):
            _m3_parity(hip, fa.AttentionShape(1, 1, 17, d), causal)


def test_m3_sequence_tile_boundaries_match_reference(hip):
    """m3_sequence_tile_boundaries_match_reference tests/wgpu_device.rs:117."""
    for s in [1, 15, 16, 17, 31, 32, 63, 64, 65, 127, 128, 129]:
        for causal in (False, True):
            _m3_parity(hip, fa.AttentionShape(1, 1, s, 32), causal)


def test_m3_multiple_batches_and_heads_match_reference(hip):
    """m3_multiple_batches_and_heads_match_reference tests/wgpu_device.rs:137."""
    for causal in (False, True):
        _m3_parity(hip, fa.AttentionShape(2, 3, 31, 16), causal)


def test_m3_large_score_range_remains_finite_and_matches_reference(hip):
    """m3_large_score_range_remains_finite_and_matches_reference tests/wgpu_device.rs:154:
    |q|, |k| ~ 7 at scale 0.125; O 8e-5 + 8e-4|e|, LSE 2e-4 + 8e-4|e|."""
    shape = fa.AttentionShape(1, 2, 31, 64)
    i = np.arange(shape.tensor_len())
    q = (np.where(i % 2 == 0, 1.0, -1.0) * (7.0 + (i % 11) * 0.125)).astype(np.float32)
    k = (np.where((i // 3) % 2 == 0, -1.0, 1.0) * (6.5 + (i % 13) * 0.1875)).astype(np.float32)
    v = (np.sin(i.astype(np.float32) * np.float32(0.03125)) * np.float32(3.0)).astype(np.float32)
    for causal in (False, True):
        _m3_parity(hip, shape, causal, (q, k, v), 0.125, ((8e-5, 8e-4), (2e-4, 8e-4)))


def test_m3_causal_future_tokens_have_zero_contribution(hip):
    """m3_causal_future_tokens_have_zero_contribution tests/wgpu_device.rs:191: K/V rows past
    the first changed to +-1000 / 500+ leave causal row 0 unchanged (O = V[0]); 1e-6."""
    shape = fa.AttentionShape(1, 1, 9, 8)
    q, k, v = _m3_fixture(shape)
    km, vm = k.copy().reshape(9, 8), v.copy().reshape(9, 8)
    km[1:] = np.where(np.arange(8) % 2 == 0, 1000.0, -1000.0)
    vm[1:] = 500.0 + np.arange(1, 9)[:, None] * 10.0 + np.arange(8)[None, :]
    ex = fa.HipFlatAttention(hip)
    cfg = fa.FlatAttentionConfig(True)
    base = ex.forward(q, k, v, shape, cfg)
    mut = ex.forward(q, km.ravel(), vm.ravel(), shape, cfg)
    assert_close("row 0 invariance", mut.output[:8], base.output[:8], 1e-6, 1e-6)
    assert_close("row 0 = V0", mut.output[:8], v[:8], 1e-6, 1e-6)
    assert_close("LSE row 0", mut.lse[:1], base.lse[:1], 1e-6, 1e-6)


# ------------------------------------------------------------------------- binary16 I/O
def _f16_fixture(shape):  # tests/wgpu_f16.rs:13
    i = np.arange(shape.tensor_len(), dtype=np.float32)
    q = (np.sin(i * np.float32(0.031) - np.float32(0.7)) * np.float32(0.85)).astype(np.float32)
    k = (np.cos(i * np.float32(0.047) + np.float32(0.2)) * np.float32(0.75)).astype(np.float32)
    v = (np.sin(i * np.float32(0.019) - np.float32(0.4)) * np.float32(1.2)).astype(np.float32)
    return q, k, v


@pytest.mark.parametrize("dims", [(1, 2, 17, 64), (1, 1, 9, 128)])
def test_f16_path_matches_reference(hip, dims):
    """packed_f16_path_is_baseline_wgsl_and_matches_reference tests/wgpu_f16.rs:104 (check_raw_
    f16_parity :67): binary16 inputs, O against the f32 oracle on the widened inputs rounded to
    binary16 (2e-3 + 5e-3|e|), LSE f32 (8e-4 + 2e-3|e|)."""
    shape = fa.AttentionShape(*dims)
    q, k, v = (x.astype(np.float16) for x in _f16_fixture(shape))
    ex = fa.HipFlatAttention(hip, fa.DTYPE_F16)
    for causal in (False, True):
        got = ex.forward(q, k, v, shape, fa.FlatAttentionConfig(causal))
        eo, el = oracle.forward(*(x.astype(np.float32) for x in (q, k, v)), *dims, causal)
        assert got.output.dtype == np.float16
        assert_close("O", got.output.astype(np.float32), eo.astype(np.float16).astype(np.float32),
                     2e-3, 5e-3)
        assert_close("LSE", got.lse, el, 8e-4, 2e-3)


def test_resident_f16_output_keeps_binary16_o_and_fp32_lse_lengths(hip):
    """resident_f16_output_keeps_binary16_o_and_fp32_lse_lengths tests/wgpu_f16.rs:212: the
    packed output holds tensor_len binary16 O values (tensor_len / 2 words) then lse_len f32."""
    shape = fa.AttentionShape(1, 1, 9, 64)
    ex = fa.HipFlatAttention(hip, fa.DTYPE_F16)
    bufs = [ex.upload(x.astype(np.float16)) for x in _f16_fixture(shape)]
    out = ex.forward_resident(*bufs, shape, fa.FlatAttentionConfig())
    lay = ex.layout(shape)
    n, m = shape.tensor_len(), shape.lse_len()
    assert lay.output_elements == n and lay.lse_elements == m
    assert lay.lse_byte_offset == n * 2 and lay.combined_bytes == (n // 2 + m) * 4
    assert out.nbytes == lay.combined_bytes
    res = ex.download_attention(out, shape)
    assert res.output.size == n and res.lse.size == m


def test_raw_f16_rejects_non_finite_input_before_dispatch(hip):
    """raw_f16_rejects_non_finite_input_before_dispatch tests/wgpu_f16.rs:249: +inf (0x7c00) at
    Q[3] is NonFiniteInput naming Q and index 3."""
    shape = fa.AttentionShape(1, 1, 1, 64)
    q = np.zeros(64, np.float16)
    q.view(np.uint16)[3] = 0x7C00
    z = np.zeros(64, np.float16)
    with pytest.raises(fa.FlatHipError) as e:
        fa.HipFlatAttention(hip, fa.DTYPE_F16).forward(q, z, z, shape, fa.FlatAttentionConfig())
    assert e.value.variant == "NonFiniteInput"
    assert "Q" in str(e.value) and "3" in str(e.value)


# --------------------------------------------------------------------- M38 property stress
def test_m38_repeated_resident_dispatch_reuses_inputs_without_numerical_drift(hip):
    """repeated_resident_dispatch_reuses_inputs_without_numerical_drift
    tests/m38_property_stress.rs:161: B1 Hq8 Hkv2 S17 D32 causal, the m38 LCG inputs, 32 resident
    forwards over the same buffers, each within 2e-4 + 1e-3|e| of the oracle (and, here, bitwise
    equal to the first)."""
    from _inputs import Lcg
    shape = fa.GroupedAttentionShape(1, 8, 2, 17, 32)
    rng = Lcg(0x4D38D15CA7C40001)
    q, k, v = rng.vec(shape.q_tensor_len()), rng.vec(shape.kv_tensor_len()), rng.vec(shape.kv_tensor_len())
    cfg = fa.FlatAttentionConfig(True)
    eo, el = oracle.forward_grouped(q, k, v, 1, 8, 2, 17, 32, True)
    ex = fa.HipRotaryGroupedAttention(hip)
    bq, bk, bv = (ex.upload(x) for x in (q, k, v))
    first = None
    for it in range(32):
        got = ex.download_attention(ex.forward_resident(bq, bk, bv, shape, cfg, None), shape)
        assert_close(f"O {it}", got.output, eo, 2e-4, 1e-3)
        assert_close(f"LSE {it}", got.lse, el, 2e-4, 1e-3)
        if first is None:
            first = got
        assert np.array_equal(got.output.view(np.uint32), first.output.view(np.uint32))


@pytest.mark.parametrize("dtype", [fa.DTYPE_F32, fa.DTYPE_BF16])
def test_m38_extreme_but_finite_scores_remain_finite_and_normalized(hip, dtype):
    """extreme_but_finite_scores_remain_finite_and_normalized tests/m38_property_stress.rs:109
    on the device: B1 Hq8 Hkv1 S33 D128, Q = +-1000, K = +-1000 (scores ~1e7), V = 1: O = 1 to
    3e-5 (f32; bf16 storage rounds O to 2^-8) and LSE finite, both masks."""
    shape = fa.GroupedAttentionShape(1, 8, 1, 33, 128)
    i = np.arange(shape.q_tensor_len())
    q = np.where(i % 2 == 0, 1000.0, -1000.0).astype(np.float32)
    j = np.arange(shape.kv_tensor_len())
    k = np.where(j % 3 == 0, -1000.0, 1000.0).astype(np.float32)
    v = np.ones(shape.kv_tensor_len(), np.float32)
    ex = fa.HipRotaryGroupedAttention(hip, dtype)
    for causal in (False, True):
        got = ex.forward(q, k, v, shape, fa.FlatAttentionConfig(causal), None)
        o = fa.storage_to_f32(got.output, dtype)
        assert np.all(np.isfinite(o)) and np.all(np.isfinite(got.lse))
        assert np.max(np.abs(o - 1.0)) <= (3e-5 if dtype == fa.DTYPE_F32 else 2 ** -8)


def test_m38_resident_kv_cache_reset_and_reuse_preserve_logical_length_contract(hip):
    """resident_kv_cache_reset_and_reuse_preserve_logical_length_contract
    tests/m38_property_stress.rs:205: capacity 8 (B1 Hkv2 D16): append 3, reset, append 2."""
    cache = fa.HipResidentKvCache(hip, 1, 2, 8, 16)
    src = lambda rows: fa.DeviceBuffer(hip, rows * 2 * 16 * 4)  # noqa: E731
    assert cache.record_append(src(3), src(3), 3) == 3
    assert len(cache) == 3 and cache.remaining_capacity() == 5
    cache.reset()
    assert cache.is_empty() and cache.remaining_capacity() == 8
    assert cache.record_append(src(2), src(2), 2) == 2
    assert len(cache) == 2 and cache.remaining_capacity() == 6


def test_m39_every_nonfinite_input_class_is_rejected(hip):
    """every_nonfinite_input_class_is_rejected tests/m39_host_api_fuzz.rs:158: NaN, +inf and -inf
    in each of Q, K, V (B1 H1 S1 D1) are NonFiniteInput naming the tensor."""
    shape = fa.AttentionShape(1, 1, 1, 1)
    ex = fa.HipFlatAttention(hip)
    for bad in (np.nan, np.inf, -np.inf):
        for t, name in enumerate("QKV"):
            x = [np.zeros(1, np.float32) for _ in range(3)]
            x[t][0] = bad
            with pytest.raises(fa.FlatHipError) as e:
                ex.forward(*x, shape, fa.FlatAttentionConfig())
            assert e.value.variant == "NonFiniteInput" and name in str(e.value), (bad, name)


def test_m19_grouped_backward_public_api_matches_oracle(hip):
    """grouped_backward_public_api_matches_oracle tests/m19_grouped_backward_api.rs:153:
    B1 Hq4 Hkv1 S5 D8, causal, scale 0.41; the forward oracle's O and LSE packed with Q, K, V,
    dO into the Q|K|V|dO|O|LSE contract, one backward encode; 4e-4 + 2e-3|e|."""
    b, hq, hkv, s, d = 1, 4, 1, 5, 8
    shape = fa.GroupedAttentionShape(b, hq, hkv, s, d)
    cfg = fa.FlatAttentionConfig(True, 0.41)
    fx = _fx(0.067, 0.75, 0.31, 0.25)
    q, k, v = fx(shape.q_tensor_len(), 0.1), fx(shape.kv_tensor_len(), 0.7), fx(shape.kv_tensor_len(), 1.3)
    do = fx(shape.q_tensor_len(), 1.9)
    eo, el = oracle.forward_grouped(q, k, v, b, hq, hkv, s, d, True, scale=0.41)
    edq, edk, edv = oracle.backward_grouped(q, k, v, do, eo, el, b, hq, hkv, s, d, True, scale=0.41)
    pipe = fa.HipGroupedBackwardRecomputePipeline(hip)
    packed = fa.DeviceBuffer.from_array(
        hip, fa.pack_grouped_backward_recompute_inputs(q, k, v, do, fa.FlatAttentionOutput(eo, el),
                                                       shape))
    grads = pipe.create_gradient_buffer(shape)
    lay = pipe.encode(packed, grads, shape, cfg)
    assert lay.kv_elements == b * hkv * s * d  # native KV-head cardinality
    g = grads.download(np.float32, lay.gradient_bytes // 4)
    for name, off, n, e in (("dQ", lay.dq_offset, lay.q_elements, edq),
                            ("dK", lay.dk_offset, lay.kv_elements, edk),
                            ("dV", lay.dv_offset, lay.kv_elements, edv)):
        assert_close(name, g[off // 4:][:n], e, 4e-4, 2e-3)
