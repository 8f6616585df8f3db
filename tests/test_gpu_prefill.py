"""GPU parity of the MFMA prefill kernels against the CPU oracle (through the C ABI).

Tolerances: f32 I/O |a-e| <= 2e-5 + 1e-4|e| for O and LSE;
16-bit I/O (f16/bf16 storage, f32 accumulation) max-abs 2e-2 after quantising the oracle's
inputs to the storage type (tests/wgpu_f16.rs:68-100 convention).
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


def _run_grouped(hip, q, k, v, shape, cfg, rot, dtype):
    ex = fa.HipRotaryGroupedAttention(hip, dtype)
    qb, kb, vb = (fa.DeviceBuffer.from_array(hip, fa.host_storage(x, dtype)) for x in (q, k, v))
    out = ex.forward_resident(qb, kb, vb, shape, cfg, rot)
    res = ex.download_attention(out, shape)
    return fa.storage_to_f32(res.output, dtype), res.lse


def _oracle_grouped(q, k, v, shape, causal, rot, units=oracle.UNIT_ALL):
    args = (q, k, v, shape.batch, shape.q_heads, shape.kv_heads, shape.seq_len, shape.head_dim,
            causal)
    if rot is None:
        return oracle.forward_grouped(*args, units=units)
    return oracle.forward_grouped_rope(*args, rot.theta, rot.position_offset, units=units)


def test_cfg1_mha_f32_causal_matches_oracle(hip):
    """MHA B1 H2 N128 D64 causal f32."""
    B, H, S, D = 1, 2, 128, 64
    q, k, v = (normal(B * H * S * D, s) for s in (11, 12, 13))
    shape = fa.AttentionShape(B, H, S, D)
    cfg = fa.FlatAttentionConfig(causal=True)
    ex = fa.HipFlatAttention(hip, fa.DTYPE_F32)
    res = ex.forward(q, k, v, shape, cfg)
    eo, el = oracle.forward(q, k, v, B, H, S, D, True)
    assert_close("O", res.output, eo, F32_ATOL, F32_RTOL)
    assert_close("LSE", res.lse, el, F32_ATOL, F32_RTOL)
    t = ex.runtime_telemetry()
    assert t.kernel_id == "PrefillMfmaF32" and t.dispatch_count == 1
    assert t.device_arch.startswith("gfx950")


@pytest.mark.parametrize("D", [32, 64, 80, 128])
@pytest.mark.parametrize("S", [1, 7, 64, 65, 130])
@pytest.mark.parametrize("causal", [False, True])
def test_mha_f32_shapes(hip, D, S, causal):
    B, H = 2, 3
    q, k, v = (normal(B * H * S * D, 100 + s + D + S) for s in range(3))
    shape = fa.GroupedAttentionShape(B, H, H, S, D)
    o, l = _run_grouped(hip, q, k, v, shape, fa.FlatAttentionConfig(causal), None, fa.DTYPE_F32)
    eo, el = _oracle_grouped(q, k, v, shape, causal, None)
    assert_close("O", o, eo, F32_ATOL, F32_RTOL)
    assert_close("LSE", l, el, F32_ATOL, F32_RTOL)


@pytest.mark.parametrize("D", [32, 64, 80, 128])
@pytest.mark.parametrize("S", [1, 7, 64, 65, 130, 300])
@pytest.mark.parametrize("causal", [False, True])
def test_mha_16bit_shapes(hip, D, S, causal):
    """The 16-bit kernel (256-row ping-pong workgroups) at edge shapes: a single key, partial
    key tiles, head dims below the padded width, and query blocks whose rows run out part-way
    through either wave group."""
    B, H = 2, 3
    q, k, v = (bf16_round(normal(B * H * S * D, 300 + s + D + S)) for s in range(3))
    shape = fa.GroupedAttentionShape(B, H, H, S, D)
    o, l = _run_grouped(hip, q, k, v, shape, fa.FlatAttentionConfig(causal), None, fa.DTYPE_BF16)
    eo, el = _oracle_grouped(q, k, v, shape, causal, None)
    assert_close("O", o, eo, H16_ATOL, 0.0)
    assert_close("LSE", l, el, H16_ATOL, 0.0)


@pytest.mark.parametrize("hq,hkv,S", [(8, 2, 65), (12, 4, 97), (32, 8, 33), (6, 1, 129)])
@pytest.mark.parametrize("causal", [False, True])
def test_gqa_rope_f16_group_shapes(hip, hq, hkv, S, causal):
    """GQA groups whose query rows (S x group) end inside a 256-row block, with RoPE, f16."""
    B, D = 2, 128
    q = f16_round(normal(B * hq * S * D, 400 + S))
    k, v = f16_round(normal(B * hkv * S * D, 401 + S)), f16_round(normal(B * hkv * S * D, 402 + S))
    shape = fa.GroupedAttentionShape(B, hq, hkv, S, D)
    rot = fa.RotaryEmbeddingConfig(1e4, 3)
    o, l = _run_grouped(hip, q, k, v, shape, fa.FlatAttentionConfig(causal), rot, fa.DTYPE_F16)
    eo, el = _oracle_grouped(q, k, v, shape, causal, rot)
    assert_close("O", o, eo, H16_ATOL, 0.0)
    assert_close("LSE", l, el, H16_ATOL, 0.0)


@pytest.mark.parametrize("dtype", [fa.DTYPE_F32, fa.DTYPE_BF16, fa.DTYPE_F16])
@pytest.mark.parametrize("hq,hkv,S", [(8, 2, 97), (32, 8, 65), (6, 1, 130)])
@pytest.mark.parametrize("causal", [False, True])
def test_gqa_without_rope_matches_grouped_oracle(hip, dtype, hq, hkv, S, causal):
    """forward_reference_grouped (src/grouped.rs:81-153): GQA with group > 1 and no RoPE
    (rotary == NULL at the C ABI), ragged S, against oracle.forward_grouped."""
    rnd = {fa.DTYPE_BF16: bf16_round, fa.DTYPE_F16: f16_round, fa.DTYPE_F32: lambda x: x}[dtype]
    atol, rtol = (F32_ATOL, F32_RTOL) if dtype == fa.DTYPE_F32 else (H16_ATOL, 0.0)
    B, D = 2, 128 if dtype != fa.DTYPE_F32 else 64
    q = rnd(normal(B * hq * S * D, 500 + S))
    k, v = rnd(normal(B * hkv * S * D, 501 + S)), rnd(normal(B * hkv * S * D, 502 + S))
    shape = fa.GroupedAttentionShape(B, hq, hkv, S, D)
    o, l = _run_grouped(hip, q, k, v, shape, fa.FlatAttentionConfig(causal), None, dtype)
    eo, el = _oracle_grouped(q, k, v, shape, causal, None)
    assert_close("O", o, eo, atol, rtol)
    assert_close("LSE", l, el, atol, rtol)
    t = hip.last_telemetry()
    assert t.kernel_id.startswith("PrefillMfma") and "PreRotatedK" not in t.kernel_id
    assert t.dispatch_count == 1  # no K rotation pass without RoPE


@pytest.mark.parametrize("hq,hkv", [(4, 4), (8, 2), (6, 1), (32, 8)])
@pytest.mark.parametrize("theta,offset", [(1e4, 0), (5e5, 37)])
def test_gqa_rope_f32(hip, hq, hkv, theta, offset):
    B, S, D = 1, 97, 64
    q = normal(B * hq * S * D, 1)
    k, v = normal(B * hkv * S * D, 2), normal(B * hkv * S * D, 3)
    shape = fa.GroupedAttentionShape(B, hq, hkv, S, D)
    rot = fa.RotaryEmbeddingConfig(theta, offset)
    for causal in (True, False):
        o, l = _run_grouped(hip, q, k, v, shape, fa.FlatAttentionConfig(causal), rot, fa.DTYPE_F32)
        eo, el = _oracle_grouped(q, k, v, shape, causal, rot)
        assert_close("O", o, eo, F32_ATOL, F32_RTOL)
        assert_close("LSE", l, el, F32_ATOL, F32_RTOL)


@pytest.mark.parametrize("dtype,rnd", [(fa.DTYPE_BF16, bf16_round), (fa.DTYPE_F16, f16_round)])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("kernel", [-1, 0])
def test_gqa_rope_16bit(hip, dtype, rnd, D, kernel):
    """kernel -1: the default main loop (assembly for bf16, D 128), 0: the HIP one."""
    hip.set_prefill_kernel(kernel)
    try:
        _gqa_rope_16bit(hip, dtype, rnd, D)
    finally:
        hip.set_prefill_kernel(-1)


def _gqa_rope_16bit(hip, dtype, rnd, D):
    B, hq, hkv, S = 2, 8, 2, 200
    q = rnd(normal(B * hq * S * D, 21))
    k, v = rnd(normal(B * hkv * S * D, 22)), rnd(normal(B * hkv * S * D, 23))
    shape = fa.GroupedAttentionShape(B, hq, hkv, S, D)
    rot = fa.RotaryEmbeddingConfig(1e4, 5)
    for causal in (True, False):
        o, l = _run_grouped(hip, q, k, v, shape, fa.FlatAttentionConfig(causal), rot, dtype)
        eo, el = _oracle_grouped(q, k, v, shape, causal, rot)
        assert_close("O", o, eo, H16_ATOL, 0.0)
        assert_close("LSE", l, el, H16_ATOL, 0.0)


def test_prerotated_and_fused_k_rotation_are_bit_identical(hip):
    B, hq, hkv, S, D = 1, 8, 2, 150, 128
    q, k, v = (bf16_round(normal(n, s)) for n, s in
               ((B * hq * S * D, 1), (B * hkv * S * D, 2), (B * hkv * S * D, 3)))
    shape = fa.GroupedAttentionShape(B, hq, hkv, S, D)
    rot = fa.RotaryEmbeddingConfig(1e4, 0)
    cfg = fa.FlatAttentionConfig(True)
    # the HIP main loop in both modes (the assembly one needs the pre-rotated K)
    hip.set_prefill_kernel(0)
    try:
        hip.set_prefill_policy(0)
        o0, l0 = _run_grouped(hip, q, k, v, shape, cfg, rot, fa.DTYPE_BF16)
        assert hip.last_telemetry().kernel_id == "PrefillMfmaBf16"
        hip.set_prefill_policy(1)
        o1, l1 = _run_grouped(hip, q, k, v, shape, cfg, rot, fa.DTYPE_BF16)
        t = hip.last_telemetry()
        assert t.kernel_id == "PrefillMfmaBf16PreRotatedK" and t.dispatch_count == 2
        assert "prefill_mfma16" in t.kernel_name
    finally:
        hip.set_prefill_policy(-1)
        hip.set_prefill_kernel(-1)
    assert np.array_equal(o0.view(np.uint32), o1.view(np.uint32))
    assert np.array_equal(l0.view(np.uint32), l1.view(np.uint32))


@pytest.mark.parametrize("kernel", [-1, 0])
def test_cfg3_full_size_bf16_gqa_rope_causal(hip, kernel):
    """BASELINE configs[2] at full size: B2 Hq32 Hkv8 N4096 D128 bf16, theta 1e4, causal.
    The oracle checks two full (batch, head) units via materialised RoPE (bit-exact to the fused
    oracle, pinned in test_oracle.py); every row is checked for finiteness and LSE bounds."""
    B, hq, hkv, S, D = 2, 32, 8, 4096, 128
    q = bf16_round(normal(B * hq * S * D, 31))
    k = bf16_round(normal(B * hkv * S * D, 32))
    v = bf16_round(normal(B * hkv * S * D, 33))
    shape = fa.GroupedAttentionShape(B, hq, hkv, S, D)
    rot = fa.RotaryEmbeddingConfig(1e4, 0)
    hip.set_prefill_kernel(kernel)
    try:
        _cfg3_full(hip, q, k, v, shape, rot)
        name = hip.last_telemetry().kernel_name
        assert ("prefill_a64" in name) == (kernel == -1), name
    finally:
        hip.set_prefill_kernel(-1)


def test_cfg3_full_size_precise_scores(hip):
    """configs[2] at full size in the precise-score mode (fa_ctx_set_prefill_precision(1)): the
    assembly kernel over K and its residual from the split rotation pass, Q split in the kernel.
    The same oracle units and V = 1 property as the default mode."""
    B, hq, hkv, S, D = 2, 32, 8, 4096, 128
    q = bf16_round(normal(B * hq * S * D, 34))
    k = bf16_round(normal(B * hkv * S * D, 35))
    v = bf16_round(normal(B * hkv * S * D, 36))
    shape = fa.GroupedAttentionShape(B, hq, hkv, S, D)
    hip.set_prefill_precision(1)
    try:
        _cfg3_full(hip, q, k, v, shape, fa.RotaryEmbeddingConfig(1e4, 0))
        t = hip.last_telemetry()
        assert "prefill_a64" in t.kernel_name and "split" in t.kernel_name, t.kernel_name
        assert t.dispatch_count == 2
    finally:
        hip.set_prefill_precision(0)


def _cfg3_full(hip, q, k, v, shape, rot):
    B, hq, hkv, S, D = shape.batch, shape.q_heads, shape.kv_heads, shape.seq_len, shape.head_dim
    o, l = _run_grouped(hip, q, k, v, shape, fa.FlatAttentionConfig(True), rot, fa.DTYPE_BF16)
    assert np.all(np.isfinite(o)) and np.all(np.isfinite(l))
    # LSE of causal row t lies in [max score, max score + ln(t+1)] -> at least >= -inf; check
    # structure on the oracle units below.
    qr = oracle.rope_rotate_rows(q, B * hq * S, 1, D, 1e4, 0, positions=np.tile(np.arange(S), B * hq))
    kr = oracle.rope_rotate_rows(k, B * hkv * S, 1, D, 1e4, 0,
                                 positions=np.tile(np.arange(S), B * hkv))
    for unit in (0, B * hq - 1):
        eo, el = oracle.forward_grouped(qr, kr, v, B, hq, hkv, S, D, True, units=(unit, unit + 1))
        sl = slice(unit * S * D, (unit + 1) * S * D)
        assert_close(f"O unit {unit}", o[sl], eo[sl], H16_ATOL, 0.0)
        ls = slice(unit * S, (unit + 1) * S)
        assert_close(f"LSE unit {unit}", l[ls], el[ls], H16_ATOL, 0.0)
    # size-independent property on every row of every unit: V = 1 gives O = 1 (the row's
    # probabilities sum to the normaliser the kernel divides by)
    ones = bf16_round(np.ones_like(v))
    o1, l1 = _run_grouped(hip, q, k, ones, shape, fa.FlatAttentionConfig(True), rot,
                          fa.DTYPE_BF16)
    assert np.max(np.abs(o1 - 1.0)) <= 2e-2
    assert np.array_equal(l1.view(np.uint32), l.view(np.uint32))


@pytest.mark.parametrize("causal", [False, True])
def test_cfg2_full_size_f32_mha(hip, causal):
    """MHA B4 H16 N2048 D128 f32; oracle on two full units."""
    B, H, S, D = 4, 16, 2048, 128
    q, k, v = (normal(B * H * S * D, 41 + s) for s in range(3))
    shape = fa.GroupedAttentionShape(B, H, H, S, D)
    o, l = _run_grouped(hip, q, k, v, shape, fa.FlatAttentionConfig(causal), None, fa.DTYPE_F32)
    for unit in (0, B * H - 1):
        eo, el = oracle.forward(q, k, v, B, H, S, D, causal, units=(unit, unit + 1))
        sl = slice(unit * S * D, (unit + 1) * S * D)
        assert_close(f"O unit {unit}", o[sl], eo[sl], F32_ATOL, F32_RTOL)
        ls = slice(unit * S, (unit + 1) * S)
        assert_close(f"LSE unit {unit}", l[ls], el[ls], F32_ATOL, F32_RTOL)
    # size-independent property on every row: V = 1 gives O = 1 exactly up to rounding
    ones = np.ones_like(v)
    o1, _ = _run_grouped(hip, q, k, ones, shape, fa.FlatAttentionConfig(causal), None, fa.DTYPE_F32)
    assert np.max(np.abs(o1 - 1.0)) <= 3e-5


@pytest.mark.parametrize("dtype,rnd,atol,rtol", [(fa.DTYPE_F32, lambda x: x, F32_ATOL, F32_RTOL),
                                                  (fa.DTYPE_BF16, bf16_round, H16_ATOL, 0.0)])
def test_projection_asymmetric_rect_and_decode(hip, dtype, rnd, atol, rtol):
    """Rectangular projection-layout GQA + RoPE (M11) incl. q_len = 1 decode and causal offset."""
    B, hq, hkv, D, theta = 2, 8, 2, 64, 1e4
    for ql, kl, off in ((1, 77, 76), (19, 90, 71), (33, 33, 0), (16, 40, 100)):
        q = rnd(normal(B * ql * hq * D, ql))
        k, v = rnd(normal(B * kl * hkv * D, kl)), rnd(normal(B * kl * hkv * D, kl + 1))
        shape = fa.AsymmetricGroupedAttentionShape(B, hq, hkv, ql, kl, D, off)
        rot = fa.AsymmetricRotaryEmbeddingConfig(theta, off + 3, 3)
        for causal in (True, False):
            pipe = fa.HipAsymmetricProjectionPipeline(hip, dtype)
            lay = pipe.layout(shape)
            out = fa.DeviceBuffer(hip, lay.combined_bytes)
            qb, kb, vb = (fa.DeviceBuffer.from_array(hip, fa.host_storage(x, dtype)) for x in (q, k, v))
            pipe.encode(qb, kb, vb, out, shape, fa.FlatAttentionConfig(causal), rot)
            res = fa.download_attention(out, lay, dtype)
            eo, el = oracle.forward_projection_asymmetric(q, k, v, B, hq, hkv, ql, kl, D, off,
                                                          causal, theta, off + 3, 3, True)
            assert_close("O", fa.storage_to_f32(res.output, dtype), eo, atol, rtol)
            assert_close("LSE", res.lse, el, atol, rtol)


def test_chunked_prefill_is_chunk_invariant_and_matches_oracle(hip):
    B, hq, hkv, S, D, theta, off = 2, 4, 2, 70, 64, 1e4, 5
    q = normal(B * S * hq * D, 1)
    k, v = normal(B * S * hkv * D, 2), normal(B * S * hkv * D, 3)
    shape = fa.GroupedAttentionShape(B, hq, hkv, S, D)
    rot = fa.RotaryEmbeddingConfig(theta, off)
    pipe = fa.HipChunkedProjectionPrefillPipeline(hip, fa.DTYPE_F32)
    qb, kb, vb = (fa.DeviceBuffer.from_array(hip, x) for x in (q, k, v))
    outs = []
    for chunk in (1, 2, 3, 16, 70, 1000):
        out = pipe.create_output_buffer(shape)
        pipe.encode(qb, kb, vb, out, shape, fa.FlatAttentionConfig(True), rot, chunk)
        outs.append(fa.download_attention(out, pipe.layout(shape), fa.DTYPE_F32))
    for r in outs[1:]:
        assert np.array_equal(r.output.view(np.uint32), outs[0].output.view(np.uint32))
        assert np.array_equal(r.lse.view(np.uint32), outs[0].lse.view(np.uint32))
    eo, el = oracle.chunked_prefill(q, k, v, B, hq, hkv, S, D, True, theta, off, 3)
    assert_close("O", outs[0].output, eo, F32_ATOL, F32_RTOL)
    assert_close("LSE", outs[0].lse, el, F32_ATOL, F32_RTOL)
    with pytest.raises(fa.FlatHipError) as e:
        pipe.encode(qb, kb, vb, out, shape, fa.FlatAttentionConfig(True), rot, 0)
    assert e.value.variant == "ZeroQueryChunkSize"


def test_chunked_prefill_precise_scores_bf16(hip):
    """Chunked prefill (causal offset = the chunk's start) in the precise-score mode at the
    assembly kernel's shape (bf16, D 128, GQA group 4): chunk sizes 64 and the whole sequence
    agree within the 16-bit bar, and match the oracle's chunked prefill."""
    B, hq, hkv, S, D, theta, off = 1, 8, 2, 300, 128, 1e4, 3
    q = bf16_round(normal(B * S * hq * D, 21))
    k, v = bf16_round(normal(B * S * hkv * D, 22)), bf16_round(normal(B * S * hkv * D, 23))
    shape = fa.GroupedAttentionShape(B, hq, hkv, S, D)
    rot = fa.RotaryEmbeddingConfig(theta, off)
    pipe = fa.HipChunkedProjectionPrefillPipeline(hip, fa.DTYPE_BF16)
    qb, kb, vb = (fa.DeviceBuffer.from_array(hip, fa.host_storage(x, fa.DTYPE_BF16))
                  for x in (q, k, v))
    outs, names = [], []
    hip.set_prefill_precision(1)
    try:
        for chunk in (64, S):
            out = pipe.create_output_buffer(shape)
            pipe.encode(qb, kb, vb, out, shape, fa.FlatAttentionConfig(True), rot, chunk)
            names.append(hip.last_telemetry().kernel_name)
            outs.append(fa.download_attention(out, pipe.layout(shape), fa.DTYPE_BF16))
    finally:
        hip.set_prefill_precision(0)
    assert all("split" in n for n in names), names
    eo, el = oracle.chunked_prefill(q, k, v, B, hq, hkv, S, D, True, theta, off, 3)
    os_ = [fa.storage_to_f32(r.output, fa.DTYPE_BF16) for r in outs]
    for o, r in zip(os_, outs):
        assert_close("O", o, eo, H16_ATOL, 0.0)
        assert_close("LSE", r.lse, el, H16_ATOL, 0.0)
    assert_close("O chunk 64 vs whole", os_[0], os_[1], H16_ATOL, 0.0)


def test_host_forward_rejects_non_finite_and_bad_lengths(hip):
    ex = fa.HipFlatAttention(hip, fa.DTYPE_F32)
    shape = fa.AttentionShape(1, 1, 4, 8)
    q = np.zeros(32, np.float32)
    k = q.copy()
    k[5] = np.inf
    with pytest.raises(fa.FlatHipError) as e:
        ex.forward(q, k, q, shape, fa.FlatAttentionConfig())
    assert e.value.variant == "NonFiniteInput" and "index 5" in str(e.value)
    with pytest.raises(fa.FlatHipError) as e:
        ex.forward(q, q[:31], q, shape, fa.FlatAttentionConfig())
    assert e.value.variant == "LengthMismatch"


def test_adversarial_scores_stay_finite(hip):
    """tests/numerical_policy.rs corpus: ties, near ties, +-7.75 cancellation, +-24 scores."""
    S, D = 16, 8
    base = np.zeros((S, D), np.float32)
    q = base.copy()
    q[:, 0] = 1.0
    cases = []
    k_tie = np.tile(np.eye(1, D, 0, np.float32), (S, 1))
    cases.append(k_tie)
    k_cancel = base.copy()
    k_cancel[:, 0] = np.where(np.arange(S) % 2 == 0, 7.75, -7.75) * np.sqrt(D)
    cases.append(k_cancel)
    k_large = base.copy()
    k_large[:, 0] = np.where(np.arange(S) % 3 == 0, 24.0, -24.0) * np.sqrt(D)
    cases.append(k_large)
    v = normal(S * D, 5)
    for kk in cases:
        for causal in (False, True):
            shape = fa.GroupedAttentionShape(1, 1, 1, S, D)
            o, l = _run_grouped(hip, q.ravel(), kk.ravel(), v, shape,
                                fa.FlatAttentionConfig(causal), None, fa.DTYPE_F32)
            eo, el = oracle.forward(q.ravel(), kk.ravel(), v, 1, 1, S, D, causal)
            assert_close("O", o, eo, F32_ATOL, F32_RTOL)
            assert_close("LSE", l, el, F32_ATOL, F32_RTOL)


@pytest.mark.parametrize("dtype,rnd", [(fa.DTYPE_BF16, bf16_round), (fa.DTYPE_F16, f16_round)])
def test_adversarial_scores_16bit(hip, dtype, rnd):
    """The 16-bit kernel's running max only moves when a tile's max exceeds it by 2^8 (log2
    units): scores rising across every key force a move on every tile, falling scores never
    move it and leave most probabilities below the 16-bit range, +-24 alternation and ties
    across several 64-key tiles and both wave groups of a 256-row workgroup."""
    S, D, H = 300, 64, 2
    idx = np.arange(S, dtype=np.float32)
    cases = {
        "rising": 0.5 * idx,
        "falling": -0.5 * idx,
        "alternating": np.where(np.arange(S) % 3 == 0, 24.0, -24.0).astype(np.float32),
        "ties": np.zeros(S, np.float32),
    }
    v = rnd(normal(H * S * D, 6))
    for name, scores in cases.items():
        q = np.zeros((H, S, D), np.float32)
        q[:, :, 0] = 1.0
        k = np.zeros((H, S, D), np.float32)
        k[:, :, 0] = scores * np.sqrt(D)
        q, k = rnd(q.ravel()), rnd(k.ravel())
        for causal in (False, True):
            shape = fa.GroupedAttentionShape(1, H, H, S, D)
            o, l = _run_grouped(hip, q, k, v, shape, fa.FlatAttentionConfig(causal), None, dtype)
            eo, el = oracle.forward(q, k, v, 1, H, S, D, causal)
            assert np.isfinite(o).all() and np.isfinite(l).all(), name
            assert_close(f"O {name}", o, eo, H16_ATOL, 0.0)
            assert_close(f"LSE {name}", l, el, H16_ATOL, 0.0)


def _rope64(x, pos, D, theta, sign):
    """Rotate [rows, D] float64 rows by sign * pos * theta^(-2j/D) (interleaved pairs)."""
    j = np.arange(D // 2)
    freq = np.float32(theta) ** (-2.0 * j / D).astype(np.float32)
    ang = sign * np.asarray(pos, np.float64)[:, None] * freq.astype(np.float64)[None, :]
    c, s = np.cos(ang), np.sin(ang)
    e, o = x[:, 0::2], x[:, 1::2]
    y = np.empty_like(x)
    y[:, 0::2] = e * c - o * s
    y[:, 1::2] = e * s + o * c
    return y


def _rope_adversarial_inputs(pattern, S, D, theta, spread):
    """Q/K whose *rotated* rows are aligned with one direction u, so the score of key t is
    sc[t] for every query: pre-rotation rows are u (or sc[t]*sqrt(D)*u) rotated back by their
    position. `spread` puts u on pair 0 only (lowest frequency: the rotation of the largest
    component is rounded in full) or across every dim."""
    u = np.zeros(D)
    if spread:
        u[:] = 1.0 / np.sqrt(D)
    else:
        u[0] = 1.0
    idx = np.arange(S, dtype=np.float64)
    sc = {"rising": 60.0 * idx / S, "falling": -60.0 * idx / S,
          "alternating": np.where(np.arange(S) % 3 == 0, 24.0, -24.0)}[pattern]
    pos = np.arange(S)
    q = _rope64(np.tile(u, (S, 1)), pos, D, theta, -1.0)
    k = _rope64(sc[:, None] * np.sqrt(D) * u[None, :], pos, D, theta, -1.0)
    return q.astype(np.float32).ravel(), k.astype(np.float32).ravel()


@pytest.mark.parametrize("pattern", ["rising", "falling", "alternating"])
@pytest.mark.parametrize("spread", [False, True])
def test_adversarial_scores_16bit_rope_prefill(hip, pattern, spread):
    """RoPE (theta 1e4, positions 0..4095) with scores rising to 60, falling to -60, or
    alternating +-24 over the whole context, through the 16-bit prefill, against the f32 oracle
    on the same bf16 inputs (tests/numerical_policy.rs:12-55 corpus, extended to RoPE).
    Precise scores (fa_ctx_set_prefill_precision(1): rotated Q and K carried as high part +
    residual) hold the 2e-2 bar on O and LSE. The default mode rounds the rotated Q and K to
    bf16 once: its score error is bounded by |s| * 2^-7 (two roundings of 2^-9 relative each,
    plus the products' rounding), which bounds the LSE error by max|s| * 2^-7."""
    S, D, theta = 4096, 128, 1e4
    q, k = _rope_adversarial_inputs(pattern, S, D, theta, spread)
    q, k = bf16_round(q), bf16_round(k)
    v = bf16_round(normal(S * D, 77))
    shape = fa.GroupedAttentionShape(1, 1, 1, S, D)
    rot = fa.RotaryEmbeddingConfig(theta, 0)
    # materialised RoPE + plain attention: bit-exact to the fused oracle (test_oracle.py)
    qr = oracle.rope_rotate_rows(q, S, 1, D, theta, 0)
    kr = oracle.rope_rotate_rows(k, S, 1, D, theta, 0)
    eo, el = oracle.forward(qr, kr, v, 1, 1, S, D, True)
    smax = float(np.max(np.abs(np.asarray(qr).reshape(S, D) @ np.asarray(kr).reshape(S, D).T
                               / np.sqrt(D))))
    try:
        hip.set_prefill_precision(1)
        o, l = _run_grouped(hip, q, k, v, shape, fa.FlatAttentionConfig(True), rot,
                            fa.DTYPE_BF16)
        assert "split" in hip.last_telemetry().kernel_name
        assert_close("O precise", o, eo, H16_ATOL, 0.0)
        assert_close("LSE precise", l, el, H16_ATOL, 0.0)
        hip.set_prefill_precision(0)
        for policy in (0, 1):
            hip.set_prefill_policy(policy)
            o, l = _run_grouped(hip, q, k, v, shape, fa.FlatAttentionConfig(True), rot,
                                fa.DTYPE_BF16)
            assert np.isfinite(o).all() and np.isfinite(l).all()
            assert_close(f"LSE default policy {policy}", l, el, smax * 2.0 ** -7, 0.0)
    finally:
        hip.set_prefill_precision(0)
        hip.set_prefill_policy(-1)


@pytest.mark.parametrize("dtype,rnd", [(fa.DTYPE_BF16, bf16_round), (fa.DTYPE_F16, f16_round)])
@pytest.mark.parametrize("hq,hkv,S,D", [(8, 2, 200, 128), (6, 1, 77, 64), (4, 4, 130, 32),
                                        (8, 2, 150, 120)])
@pytest.mark.parametrize("causal", [False, True])
def test_precise_rope_prefill_matches_oracle(hip, dtype, rnd, hq, hkv, S, D, causal):
    """The split-score kernel (precision mode 1) at edge shapes: ragged key tiles, GQA groups,
    head dims below the padded width, both 16-bit formats, a RoPE offset."""
    B = 2
    q = rnd(normal(B * hq * S * D, 600 + S + D))
    k, v = rnd(normal(B * hkv * S * D, 601 + S)), rnd(normal(B * hkv * S * D, 602 + S))
    shape = fa.GroupedAttentionShape(B, hq, hkv, S, D)
    rot = fa.RotaryEmbeddingConfig(1e4, 9)
    try:
        hip.set_prefill_precision(1)
        o, l = _run_grouped(hip, q, k, v, shape, fa.FlatAttentionConfig(causal), rot, dtype)
        t = hip.last_telemetry()
        # bf16 at D 128 with a power-of-two group: the assembly kernel after the split K
        # rotation (two dispatches); otherwise the HIP kernel rotating K on load (one)
        assert "split" in t.kernel_name
        assert t.dispatch_count == (2 if "prefill_a64" in t.kernel_name else 1), t.kernel_name
    finally:
        hip.set_prefill_precision(0)
    eo, el = _oracle_grouped(q, k, v, shape, causal, rot)
    assert_close("O", o, eo, H16_ATOL, 0.0)
    assert_close("LSE", l, el, H16_ATOL, 0.0)


@pytest.mark.parametrize("dtype,rnd,atol,rtol", [(fa.DTYPE_BF16, bf16_round, H16_ATOL, 0.0),
                                                  (fa.DTYPE_F32, lambda x: x, F32_ATOL, F32_RTOL)])
def test_prepared_forward_matches_one_shot_and_oracle(hip, dtype, rnd, atol, rtol):
    """PreparedGroupedForward::prepare / encode_prepared (src/wgpu_forward_grouped.rs:352,496):
    prepare binds the buffers and owns the RoPE table and K rotation workspace; repeated
    launches, with the inputs' contents changed in between, give bitwise the one-shot call's
    results; a prepared forward is rejected by another context (ForeignBuffer)."""
    B, hq, hkv, S, D = 2, 8, 2, 150, 128
    shape = fa.GroupedAttentionShape(B, hq, hkv, S, D)
    rot = fa.RotaryEmbeddingConfig(1e4, 7)
    cfg = fa.FlatAttentionConfig(True)
    ex = fa.HipRotaryGroupedAttention(hip, dtype)
    ins = [[rnd(normal(n, s0 + i)) for i, n in enumerate(
        (B * hq * S * D, B * hkv * S * D, B * hkv * S * D))] for s0 in (61, 71)]
    qb, kb, vb = (fa.DeviceBuffer.from_array(hip, fa.host_storage(x, dtype)) for x in ins[0])
    out = fa.DeviceBuffer(hip, ex.layout(shape).combined_bytes)
    prep = ex.prepare(qb, kb, vb, out, shape, cfg, rot)
    assert prep.layout() == ex.layout(shape)
    for q, k, v in ins + ins[:1]:
        for buf, x in zip((qb, kb, vb), (q, k, v)):
            buf.upload(fa.host_storage(x, dtype))
        ex.encode_prepared(prep)
        got = ex.download_attention(out, shape)
        one = _run_grouped(hip, q, k, v, shape, cfg, rot, dtype)
        assert np.array_equal(fa.storage_to_f32(got.output, dtype).view(np.uint32),
                              one[0].view(np.uint32))
        assert np.array_equal(got.lse.view(np.uint32), one[1].view(np.uint32))
        eo, el = _oracle_grouped(q, k, v, shape, True, rot, units=(0, 1))
        assert_close("O unit 0", fa.storage_to_f32(got.output, dtype)[:S * D], eo[:S * D], atol,
                     rtol)
        assert_close("LSE unit 0", got.lse[:S], el[:S], atol, rtol)
    other = fa.HipContext(0)
    try:
        with pytest.raises(fa.FlatHipError) as e:
            fa.HipRotaryGroupedAttention(other, dtype).encode_prepared(prep)
        assert e.value.variant == "ForeignBuffer"
    finally:
        other.close()
    prep.release()


@pytest.mark.parametrize("kernel", [-1, 1])
@pytest.mark.parametrize("where", ["q", "k", "v"])
def test_nan_in_device_resident_input_stays_in_its_rows(hip, kernel, where):
    """A NaN inside a device-resident input (the host validation of fa_forward_gqa_rope_host
    never sees it). prefill.hip is compiled with -fno-honor-nans, so the compiler may assume no
    NaN reaches its max/compare operations; this pins what the kernels return then.
    * Q element of row r: row r's O and LSE are NaN, every other row is bitwise unchanged.
    * K element of key j: O and LSE of every query row of that kv head's group at t >= j are
      NaN (masked scores are replaced, so rows t < j are bitwise unchanged).
    * V element (j, d): O[:, d] of that group's rows t >= j is NaN, LSE and every other dim
      unchanged. Rows t < j of a query block whose key range reaches j's 64-key tile may also
      come back NaN in dim d: their masked probabilities enter the P.V product as zeros, and
      0 * NaN is NaN. Rows of blocks that stop before that tile are bitwise unchanged.
    kernel -1 is the HIP main loop, 1 the assembly one; both use 256-row query blocks, i.e.
    128 positions of a group of 2."""
    B, hq, hkv, S, D = 1, 4, 2, 300, 128
    q, k, v = (fa.host_storage(bf16_round(normal(n, s)), fa.DTYPE_BF16) for n, s in
               ((B * hq * S * D, 51), (B * hkv * S * D, 52), (B * hkv * S * D, 53)))
    shape = fa.GroupedAttentionShape(B, hq, hkv, S, D)
    rot = fa.RotaryEmbeddingConfig(1e4, 0)
    cfg = fa.FlatAttentionConfig(True)
    ex = fa.HipRotaryGroupedAttention(hip, fa.DTYPE_BF16)

    def run(qs, ks, vs):
        bufs = [fa.DeviceBuffer.from_array(hip, x) for x in (qs, ks, vs)]
        res = ex.download_attention(ex.forward_resident(*bufs, shape, cfg, rot), shape)
        return (fa.storage_to_f32(res.output, fa.DTYPE_BF16).reshape(hq, S, D),
                res.lse.reshape(hq, S))

    nan = np.uint16(0x7FC0)
    hit_o = np.zeros((hq, S, D), bool)   # must be NaN
    free_o = np.zeros((hq, S, D), bool)  # not asserted
    hit_l = np.zeros((hq, S), bool)
    q2, k2, v2 = q.copy(), k.copy(), v.copy()
    if where == "q":
        q2[(1 * S + 40) * D + 5] = nan
        hit_o[1, 40, :] = hit_l[1, 40] = True
    elif where == "k":
        k2[(0 * S + 70) * D + 3] = nan
        hit_o[0:2, 70:, :] = True
        hit_l[0:2, 70:] = True
    else:
        v2[(1 * S + 250) * D + 9] = nan
        hit_o[2:4, 250:, 9] = True
        free_o[2:4, 128:250, 9] = True
    hip.set_prefill_kernel(kernel)
    try:
        o0, l0 = run(q, k, v)
        o1, l1 = run(q2, k2, v2)
        if kernel == 1:
            assert "prefill_a64" in hip.last_telemetry().kernel_name
    finally:
        hip.set_prefill_kernel(-1)
    keep = ~(hit_o | free_o)
    assert np.array_equal(o1[keep].view(np.uint32), o0[keep].view(np.uint32))
    assert np.array_equal(l1[~hit_l].view(np.uint32), l0[~hit_l].view(np.uint32))
    assert np.isnan(o1[hit_o]).all(), f"{np.isnan(o1[hit_o]).sum()} of {hit_o.sum()} NaN"
    assert np.isnan(l1[hit_l]).all(), f"{np.isnan(l1[hit_l]).sum()} of {hit_l.sum()} NaN"
