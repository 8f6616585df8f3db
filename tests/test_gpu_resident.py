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
