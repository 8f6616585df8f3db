"""GPU parity of the fixed-capacity resident KV cache (WgpuResidentKvCache,
src/wgpu_kv_cache.rs) and the q_len = 1 resident decode (WgpuResidentDecodePipeline,
src/wgpu_decode.rs).

Appends are checked byte-exactly against the host rows; decode against the C oracle's paged
decode (pool = the resident buffers, one `capacity`-row page per batch element).
Numerics: f32 2e-5 + 1e-4|e|; bf16 2e-2.
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


def _oracle_resident(q, k, v, batch, capacity, kv_len, hq, hkv, D, q_pos, theta=1e4):
    bt = np.arange(batch, dtype=np.int32).reshape(batch, 1)
    return oracle.paged_decode(q, k, v, batch, capacity, bt, [kv_len] * batch, hq, hkv, D, True,
                               theta, q_positions=[q_pos] * batch)


def test_resident_cache_appends_in_place_and_decode_matches_oracle(hip):
    """Two appends land after the live prefix of every batch element (sentinel-filled rows past
    the live length stay untouched); decode over the cache (encode :265) matches the oracle."""
    batch, hkv, cap, D, hq = 3, 2, 100, 64, 4
    width = hkv * D
    cache = fa.HipResidentKvCache(hip, batch, hkv, cap, D, fa.DTYPE_F32)
    kb, vb = cache.k_buffer(), cache.v_buffer()
    kb.upload(np.full(batch * cap * width, 17.0, np.float32))
    vb.upload(np.full(batch * cap * width, -19.0, np.float32))
    expect_k = np.full((batch, cap, width), 17.0, np.float32)
    expect_v = np.full((batch, cap, width), -19.0, np.float32)
    live = 0
    for n, seed in ((37, 1), (25, 2)):
        ks = normal(batch * n * width, seed).reshape(batch, n, width)
        vs = normal(batch * n * width, seed + 10).reshape(batch, n, width)
        got = cache.record_append(fa.DeviceBuffer.from_array(hip, ks),
                                  fa.DeviceBuffer.from_array(hip, vs), n)
        expect_k[:, live:live + n] = ks
        expect_v[:, live:live + n] = vs
        live += n
        assert got == live == len(cache)
    assert cache.remaining_capacity() == cap - live
    k_dev = kb.download(np.float32, batch * cap * width)
    v_dev = vb.download(np.float32, batch * cap * width)
    assert np.array_equal(k_dev.view(np.uint32), expect_k.reshape(-1).view(np.uint32))
    assert np.array_equal(v_dev.view(np.uint32), expect_v.reshape(-1).view(np.uint32))

    q = normal(batch * hq * D, 3)
    pipe = fa.HipResidentDecodePipeline(hip, fa.DTYPE_F32)
    out = pipe.create_output_buffer(cache, hq)
    lay = pipe.encode(fa.DeviceBuffer.from_array(hip, q), cache, out, hq,
                      fa.FlatAttentionConfig(True), 1e4, live - 1)
    res = fa.download_attention(out, lay, fa.DTYPE_F32)
    eo, el = _oracle_resident(q, k_dev, v_dev, batch, cap, live, hq, hkv, D, live - 1)
    assert_close("O", res.output, eo, F32_ATOL, F32_RTOL)
    assert_close("LSE", res.lse, el, F32_ATOL, F32_RTOL)

    with pytest.raises(fa.FlatHipError) as e:
        cache.record_append(fa.DeviceBuffer.from_array(hip, np.zeros(batch * 39 * width, np.float32)),
                            fa.DeviceBuffer.from_array(hip, np.zeros(batch * 39 * width, np.float32)),
                            39)
    assert e.value.variant == "CapacityExceeded"
    assert "append 39 at length 62 exceeds capacity 100" in str(e.value)
    assert len(cache) == live
    cache.reset()
    assert len(cache) == 0


@pytest.mark.parametrize("dtype", [fa.DTYPE_BF16, fa.DTYPE_F16, fa.DTYPE_F32])
@pytest.mark.parametrize("batch,hq,hkv,cap,kv_len,D",
                         [(1, 16, 4, 8192, 8192, 64), (4, 32, 8, 1024, 777, 128),
                          (2, 8, 8, 48, 17, 64)])
def test_external_pre_rotated_k_decode_matches_oracle(hip, dtype, batch, hq, hkv, cap, kv_len, D):
    """encode_external_pre_rotated_k :301 over framework-owned [batch, capacity, Hkv*D] buffers;
    row 1 is the published M15/M48 decode shape (B1 Hq16 Hkv4 D64, kv 8192)."""
    rng = np.random.default_rng(batch * 1000 + kv_len)
    width = hkv * D
    rnd = {fa.DTYPE_BF16: bf16_round, fa.DTYPE_F16: f16_round}.get(dtype, lambda x: x)
    k = rnd(normal(batch * cap * width, int(rng.integers(1 << 30))))
    v = rnd(normal(batch * cap * width, int(rng.integers(1 << 30))))
    q = rnd(normal(batch * hq * D, int(rng.integers(1 << 30))))
    q_pos = kv_len + 5
    shape = fa.AsymmetricGroupedAttentionShape(batch, hq, hkv, 1, kv_len, D, q_pos)
    pipe = fa.HipResidentDecodePipeline(hip, dtype)
    out = fa.DeviceBuffer(hip, pipe.layout(batch, hq, D).combined_bytes)
    bufs = [fa.DeviceBuffer.from_array(hip, fa.host_storage(x, dtype)) for x in (q, k, v)]
    lay = pipe.encode_external_pre_rotated_k(bufs[0], bufs[1], bufs[2], out, shape,
                                             fa.FlatAttentionConfig(True),
                                             fa.AsymmetricRotaryEmbeddingConfig(1e4, q_pos, 0), cap)
    res = fa.download_attention(out, lay, dtype)
    eo, el = _oracle_resident(q, k, v, batch, cap, kv_len, hq, hkv, D, q_pos)
    o = fa.storage_to_f32(res.output, dtype)
    if dtype == fa.DTYPE_F32:
        assert_close("O", o, eo, F32_ATOL, F32_RTOL)
        assert_close("LSE", res.lse, el, F32_ATOL, F32_RTOL)
    else:
        assert_close("O", o, eo, H16_ATOL, 0.0)
        assert_close("LSE", res.lse, el, H16_ATOL, 0.0)
    t = hip.last_telemetry()
    want = "DecodePagedMfma" if dtype != fa.DTYPE_F32 and cap % 16 == 0 else "DecodePagedSplitK"
    assert t.kernel_id == want


def test_external_decode_rejects_invisible_rows_and_query_len(hip):
    pipe = fa.HipResidentDecodePipeline(hip, fa.DTYPE_F32)
    buf = fa.DeviceBuffer(hip, 1 << 20)
    with pytest.raises(fa.FlatHipError) as e:
        pipe.encode_external_pre_rotated_k(
            buf, buf, buf, buf, fa.AsymmetricGroupedAttentionShape(1, 2, 1, 1, 40, 64, 20),
            fa.FlatAttentionConfig(True), fa.AsymmetricRotaryEmbeddingConfig(1e4, 39, 0), 64)
    assert e.value.variant == "CausalVisibilityMismatch"
    with pytest.raises(fa.FlatHipError) as e:
        pipe.encode_external_pre_rotated_k(
            buf, buf, buf, buf, fa.AsymmetricGroupedAttentionShape(1, 2, 1, 2, 40, 64, 39),
            fa.FlatAttentionConfig(True), fa.AsymmetricRotaryEmbeddingConfig(1e4, 39, 0), 64)
    assert e.value.variant == "LengthMismatch"


def _m15_fixture(n, phase):
    x = np.arange(n, dtype=np.float32) * np.float32(0.023) + np.float32(phase)
    return (np.sin(x) * 1.125 + np.cos(x * np.float32(0.29)) * 0.4375).astype(np.float32)


def test_one_pipeline_tracks_token_by_token_cache_growth(hip):
    """tests/m15_growing_cache.rs:146: one pipeline and one output buffer serve a capacity-6
    cache grown one pre-rotated K row at a time; after every append the decode at the newest
    position matches the raw-K asymmetric RoPE oracle (projection_asymmetric.rs:97)."""
    hq, hkv, cap, D, theta = 4, 1, 6, 32, 1e4
    cache = fa.HipResidentKvCache(hip, 1, hkv, cap, D, fa.DTYPE_F32)
    pipe = fa.HipResidentDecodePipeline(hip, fa.DTYPE_F32)
    out = None
    raw_k, vs = [], []
    for pos in range(cap):
        k_row = _m15_fixture(D, 0.4 + pos * 0.13)
        v_row = _m15_fixture(D, 1.1 + pos * 0.17)
        raw_k.append(k_row)
        vs.append(v_row)
        rot = oracle.rope_rotate_rows(k_row, 1, hkv, D, theta, position_offset=pos)
        assert cache.record_append(fa.DeviceBuffer.from_array(hip, rot),
                                   fa.DeviceBuffer.from_array(hip, v_row), 1) == pos + 1
        assert len(cache) == pos + 1
        if out is None:
            out = pipe.create_output_buffer(cache, hq)
        q = _m15_fixture(hq * D, 2.0 + pos * 0.19)
        lay = pipe.encode(fa.DeviceBuffer.from_array(hip, q), cache, out, hq,
                          fa.FlatAttentionConfig(True), theta, pos)
        res = fa.download_attention(out, lay, fa.DTYPE_F32)
        eo, el = oracle.forward_projection_asymmetric(
            q, np.concatenate(raw_k), np.concatenate(vs), 1, hq, hkv, 1, pos + 1, D, pos, True,
            theta=theta, q_rope_offset=pos, kv_rope_offset=0)
        assert_close(f"O@{pos}", res.output, eo, 2e-4, 1e-3)
        assert_close(f"LSE@{pos}", res.lse, el, 2e-4, 1e-3)
    assert cache.remaining_capacity() == 0


def _m48_fixture(n, phase):
    x = np.arange(n, dtype=np.float32) * np.float32(0.021) + np.float32(phase)
    return (np.sin(x) * 1.75 + np.cos(x * np.float32(0.43)) * 0.34375).astype(np.float32)


@pytest.mark.parametrize("dtype", [fa.DTYPE_F32, fa.DTYPE_BF16, fa.DTYPE_F16])
@pytest.mark.parametrize("batch,hq,hkv,kv_len,D,causal_pos,q_rope,causal", [
    (1, 16, 4, 192, 64, 191, 191, True),   # m48_sciagent_decode_matches_oracle :105
    (1, 16, 4, 16, 64, 7, 7, True),        # m48_causal_offset_masks_future_kv :179
    (3, 32, 4, 777, 128, 900, 1234, True),  # past the end: every key visible
    (2, 8, 2, 300, 64, 120, 40, True),     # causal and RoPE positions differ
    (2, 12, 2, 33, 32, 0, 5, False),
    (1, 4, 2, 9, 6, 8, 8, True),           # f32 head_dim 6: the prefill-kernel route
    (1, 16, 4, 8192, 64, 8191, 8191, True),  # the published M48 shape (bench line)
])
def test_m48_decode_kv_reuse_matches_oracle(hip, dtype, batch, hq, hkv, kv_len, D, causal_pos,
                                            q_rope, causal):
    """encode_pre_rotated_k_decode_kv_reuse src/wgpu_external_asymmetric.rs:216 against the
    raw-K asymmetric oracle (projection_asymmetric.rs:97) with K rotated on the host as the
    reference's test does (tests/m48_decode_kv_reuse.rs:21); causal masking keeps keys up to the
    shape's query position. Tolerance: f32 1.5e-4 + 1e-3|e| (the reference's), 16-bit 2e-2 on
    inputs rounded to the storage type."""
    if D % 8 and dtype != fa.DTYPE_F32:
        pytest.skip("16-bit storage needs head_dim % 8 == 0")
    rnd = {fa.DTYPE_BF16: bf16_round, fa.DTYPE_F16: f16_round}.get(dtype, lambda x: x)
    width = hkv * D
    q = rnd(_m48_fixture(batch * hq * D, 0.2))
    raw_k = _m48_fixture(batch * kv_len * width, 0.8)
    v = rnd(_m48_fixture(batch * kv_len * width, 1.4))
    k = np.concatenate([oracle.rope_rotate_rows(raw_k.reshape(batch, -1)[b], kv_len, hkv, D, 1e4)
                        for b in range(batch)])
    k = rnd(k)
    shape = fa.AsymmetricGroupedAttentionShape(batch, hq, hkv, 1, kv_len, D, causal_pos)
    rot = fa.AsymmetricRotaryEmbeddingConfig(1e4, q_rope, 0)
    pipe = fa.HipAsymmetricProjectionPipeline.with_decode_kv_reuse(hip, True, dtype)
    out = pipe.create_output_buffer(shape)
    bufs = [fa.DeviceBuffer.from_array(hip, fa.host_storage(x, dtype)) for x in (q, k, v)]
    lay = pipe.encode_pre_rotated_k_decode_kv_reuse(bufs[0], bufs[1], bufs[2], out, shape,
                                                    fa.FlatAttentionConfig(causal), rot)
    res = fa.download_attention(out, lay, dtype)
    eo, el = oracle.forward_projection_asymmetric(
        q, k, v, batch, hq, hkv, 1, kv_len, D, causal_pos, causal, theta=1e4, q_rope_offset=q_rope,
        rotate_k=False)
    o = fa.storage_to_f32(res.output, dtype)
    if dtype == fa.DTYPE_F32:
        assert_close("O", o, eo, 1.5e-4, 1e-3)
        assert_close("LSE", res.lse, el, 1.5e-4, 1e-3)
    else:
        assert_close("O", o, eo, H16_ATOL, 0.0)
        assert_close("LSE", res.lse, el, H16_ATOL, 0.0)
    kid = hip.last_telemetry().kernel_id
    if D % 4:
        assert kid.startswith("Prefill")
    else:
        assert kid == ("DecodePagedMfma" if dtype != fa.DTYPE_F32 and kv_len % 16 == 0
                       else "DecodePagedSplitK")
    if causal and causal_pos == 7 and kv_len == 16 and dtype == fa.DTYPE_F32:
        # the reference's own oracle anchor for the masking: the first 8 keys alone
        eo8, el8 = oracle.forward_projection_asymmetric(
            q, k.reshape(kv_len, width)[:8].reshape(-1), v.reshape(kv_len, width)[:8].reshape(-1),
            1, hq, hkv, 1, 8, D, 7, False, theta=1e4, q_rope_offset=7, rotate_k=False)
        assert_close("O(8 keys)", o, eo8, 1.5e-4, 1e-3)


def test_m48_is_opt_in_and_baseline_routes_unchanged(hip):
    """m48_is_opt_in tests/m48_decode_kv_reuse.rs:318; encode_pre_rotated_k on a pipeline with the
    candidate keeps its prefill route (with_decode_kv_reuse :78)."""
    shape = fa.AsymmetricGroupedAttentionShape(1, 16, 4, 1, 1, 64, 0)
    rot = fa.AsymmetricRotaryEmbeddingConfig(1e4, 0, 0)
    zq = fa.DeviceBuffer.from_array(hip, np.zeros(16 * 64, np.float32))
    zkv = fa.DeviceBuffer.from_array(hip, np.zeros(4 * 64, np.float32))
    base = fa.HipAsymmetricProjectionPipeline(hip)
    out = base.create_output_buffer(shape)
    with pytest.raises(fa.FlatHipError) as e:
        base.encode_pre_rotated_k_decode_kv_reuse(zq, zkv, zkv, out, shape,
                                                  fa.FlatAttentionConfig(True), rot)
    assert e.value.variant == "CandidateNotEnabled"
    cand = fa.HipAsymmetricProjectionPipeline.with_decode_kv_reuse(hip, True)
    cand.encode_pre_rotated_k(zq, zkv, zkv, out, shape, fa.FlatAttentionConfig(True), rot)
    assert hip.last_telemetry().kernel_id.startswith("Prefill")
