"""GPU parity of the recompute backward (M19-M21, WgpuGroupedBackwardRecomputePipeline,
src/wgpu_backward_grouped.rs) against the CPU oracle (backward_reference_grouped,
src/backward_grouped.rs:17).

Cases follow the reference's GPU tests: the M19 GQA/MQA pair (tests/m19_grouped_backward_wgpu.rs,
tolerance 4e-4 + 2e-3|e|), the M20 stress matrix with three repeated encodes
(tests/m20_grouped_backward_stress.rs, 5e-4 + 2.5e-3|e|) and the M21 prepared-reuse cases with
four encode_prepared calls (tests/m21_prepared_grouped_backward_reuse.rs, 4e-4 + 2e-3|e|), then
tile-crossing sequence lengths and head dims up to 128, 16-bit storage, bitwise determinism and
the separate-tensor entry fed by this library's own forward.

16-bit storage: the oracle runs on the bf16/f16-rounded inputs (and the forward it was given);
the kernel rounds P and dS to the storage type for the MFMA products and stores gradients in it,
so the bound is 2e-2 of the tensor's largest magnitude plus 2e-2|e|.
"""
import numpy as np
import pytest

import oracle
from _inputs import bf16_round, f16_round, normal
from conftest import assert_close

import flat_attention_amd as fa

pytestmark = pytest.mark.gpu


def _fx(n, phase, step, a, b, w):
    x = np.arange(n, dtype=np.float32) * np.float32(step) + np.float32(phase)
    return (np.sin(x) * np.float32(a) + np.cos(x * np.float32(w)) * np.float32(b)).astype(np.float32)


def fx_m19(n, phase):  # tests/m19_grouped_backward_wgpu.rs:49
    return _fx(n, phase, 0.071, 0.75, 0.25, 0.37)


def fx_m20(n, phase):  # tests/m20_grouped_backward_stress.rs:49
    return _fx(n, phase, 0.031, 0.63, 0.37, 0.47)


def fx_m21(n, phase):  # tests/m21_prepared_grouped_backward_reuse.rs:48
    return _fx(n, phase, 0.053, 0.7, 0.3, 0.37)


def _expected(q, k, v, do, shape, causal, scale):
    s = shape
    o, lse = oracle.forward_grouped(q, k, v, s.batch, s.q_heads, s.kv_heads, s.seq_len,
                                    s.head_dim, causal, scale)
    grads = oracle.backward_grouped(q, k, v, do, o, lse, s.batch, s.q_heads, s.kv_heads,
                                    s.seq_len, s.head_dim, causal, scale, threads=8)
    return fa.FlatAttentionOutput(o, lse), grads


def _check(tag, got, want, atol, rtol):
    for name, a, e in zip(("dQ", "dK", "dV"), (got.dq, got.dk, got.dv), want):
        assert_close(f"{tag}-{name}", a, e, atol, rtol)


def _packed_case(hip, shape, config, fixture, phases, repeats, atol, rtol, prepared=False):
    q = fixture(shape.q_tensor_len(), phases[0])
    k = fixture(shape.kv_tensor_len(), phases[1])
    v = fixture(shape.kv_tensor_len(), phases[2])
    do = fixture(shape.q_tensor_len(), phases[3])
    fwd, want = _expected(q, k, v, do, shape, config.causal, config.softmax_scale)
    pipe = fa.HipGroupedBackwardRecomputePipeline(hip, fa.DTYPE_F32)
    packed = fa.pack_grouped_backward_recompute_inputs(q, k, v, do, fwd, shape)
    fbuf = fa.DeviceBuffer.from_array(hip, packed)
    gbuf = pipe.create_gradient_buffer(shape)
    prep = pipe.prepare(fbuf, gbuf, shape, config) if prepared else None
    for rep in range(repeats):
        gbuf.fill_u32(0x7FC00000)  # NaN: every gradient element must be written
        lay = pipe.encode_prepared(prep) if prepared else pipe.encode(fbuf, gbuf, shape, config)
        assert lay == pipe.layout(shape)
        got = pipe.download_gradients(gbuf, shape)
        _check(f"{shape}-causal{config.causal}-rep{rep}", got, want, atol, rtol)
    tele = hip.last_telemetry()
    assert tele.kernel_id == "BackwardRecompute" and tele.dispatch_count == 3
    fbuf.free()
    gbuf.free()


@pytest.mark.parametrize("kv_heads,causal", [(2, True), (1, False)])
def test_m19_gqa_mqa_matches_oracle(hip, kv_heads, causal):
    shape = fa.GroupedAttentionShape(2, 4, kv_heads, 5, 8)
    _packed_case(hip, shape, fa.FlatAttentionConfig(causal, 0.41), fx_m19,
                 (0.1, 0.7, 1.3, 1.9), 1, 4e-4, 2e-3)


M20_CASES = [((1, 1, 1, 1, 2), False, None), ((1, 4, 4, 3, 8), True, None),
             ((2, 8, 2, 5, 16), False, 0.23), ((1, 8, 1, 9, 32), True, 0.17),
             ((2, 12, 3, 7, 6), True, None)]


@pytest.mark.parametrize("idx", range(len(M20_CASES)))
def test_m20_stress_matrix_repeated(hip, idx):
    dims, causal, scale = M20_CASES[idx]
    ph = idx * 0.37
    _packed_case(hip, fa.GroupedAttentionShape(*dims), fa.FlatAttentionConfig(causal, scale),
                 fx_m20, (ph + 0.1, ph + 0.7, ph + 1.3, ph + 1.9), 3, 5e-4, 2.5e-3)


@pytest.mark.parametrize("dims,causal,scale", [((1, 4, 4, 7, 8), True, None),
                                               ((1, 8, 2, 9, 16), False, 0.27),
                                               ((2, 4, 1, 5, 12), True, 0.31)])
def test_m21_prepared_reuse(hip, dims, causal, scale):
    _packed_case(hip, fa.GroupedAttentionShape(*dims), fa.FlatAttentionConfig(causal, scale),
                 fx_m21, (0.1, 0.7, 1.3, 1.9), 4, 4e-4, 2e-3, prepared=True)


# Tile edges: 64-row staged tiles, 128-row workgroups, 32-row waves; head dims padded to 32/64/128.
@pytest.mark.parametrize("dims,causal", [
    ((1, 4, 2, 130, 64), True), ((1, 4, 2, 130, 64), False), ((2, 2, 1, 257, 128), True),
    ((1, 8, 8, 64, 128), False), ((1, 6, 2, 200, 96), True), ((1, 2, 1, 33, 40), True),
    ((1, 4, 1, 129, 20), False), ((1, 4, 2, 96, 7), True)])
def test_f32_tile_edges(hip, dims, causal):
    shape = fa.GroupedAttentionShape(*dims)
    B, Hq, Hkv, S, D = dims
    q, k, v, do = (normal(n, 11 + i) for i, n in enumerate(
        (B * Hq * S * D, B * Hkv * S * D, B * Hkv * S * D, B * Hq * S * D)))
    _packed_case(hip, shape, fa.FlatAttentionConfig(causal), lambda n, p: (q, k, v, do)[int(p)],
                 (0, 1, 2, 3), 1, 5e-4, 2.5e-3)


@pytest.mark.parametrize("dtype", [fa.DTYPE_BF16, fa.DTYPE_F16])
@pytest.mark.parametrize("dims,causal", [((1, 8, 2, 256, 128), True),
                                         ((2, 4, 4, 130, 64), False),
                                         ((1, 4, 1, 77, 32), True)])
def test_16bit_storage(hip, dtype, dims, causal):
    rnd = bf16_round if dtype == fa.DTYPE_BF16 else f16_round
    shape = fa.GroupedAttentionShape(*dims)
    B, Hq, Hkv, S, D = dims
    q, k, v, do = (rnd(normal(n, 21 + i)) for i, n in enumerate(
        (B * Hq * S * D, B * Hkv * S * D, B * Hkv * S * D, B * Hq * S * D)))
    fwd, want = _expected(q, k, v, do, shape, causal, None)
    fwd = fa.FlatAttentionOutput(rnd(fwd.output), fwd.lse)
    # the oracle's gradients for the rounded O the kernel is given
    want = oracle.backward_grouped(q, k, v, do, fwd.output, fwd.lse, B, Hq, Hkv, S, D, causal,
                                   threads=8)
    pipe = fa.HipGroupedBackwardRecomputePipeline(hip, dtype)
    got = pipe.backward(q, k, v, do, fwd, shape, fa.FlatAttentionConfig(causal))
    for name, a, e in zip(("dQ", "dK", "dV"), (got.dq, got.dk, got.dv), want):
        assert_close(name, a, e, 2e-2 * float(np.abs(e).max()), 2e-2)


def test_deterministic_bitwise(hip):
    shape = fa.GroupedAttentionShape(1, 8, 2, 300, 128)
    B, Hq, Hkv, S, D = 1, 8, 2, 300, 128
    q, k, v, do = (bf16_round(normal(n, 31 + i)) for i, n in enumerate(
        (B * Hq * S * D, B * Hkv * S * D, B * Hkv * S * D, B * Hq * S * D)))
    fwd, _ = _expected(q, k, v, do, shape, True, None)
    pipe = fa.HipGroupedBackwardRecomputePipeline(hip, fa.DTYPE_BF16)
    packed = fa.pack_grouped_backward_recompute_inputs(q, k, v, do, fwd, shape, fa.DTYPE_BF16)
    fbuf = fa.DeviceBuffer.from_array(hip, packed)
    lay = pipe.layout(shape)
    outs = []
    for _ in range(3):
        g = pipe.create_gradient_buffer(shape)
        pipe.encode(fbuf, g, shape, fa.FlatAttentionConfig(True))
        outs.append(g.download(np.uint8, lay.gradient_bytes))
        g.free()
    assert all(np.array_equal(outs[0], o) for o in outs[1:])


@pytest.mark.parametrize("dtype", [fa.DTYPE_F32, fa.DTYPE_BF16])
def test_training_chain_own_forward(hip, dtype):
    """Forward (fa_forward_gqa_rope, no RoPE) -> backward (fa_backward_grouped) over the forward's
    own packed O|LSE, like tests/m23_wgpu_training_chain.rs; checked against the oracle given the
    same O and LSE."""
    B, Hq, Hkv, S, D = 2, 8, 2, 192, 64
    rnd = (lambda x: x) if dtype == fa.DTYPE_F32 else bf16_round
    q, k, v, do = (rnd(normal(n, 41 + i)) for i, n in enumerate(
        (B * Hq * S * D, B * Hkv * S * D, B * Hkv * S * D, B * Hq * S * D)))
    shape = fa.GroupedAttentionShape(B, Hq, Hkv, S, D)
    cfg = fa.FlatAttentionConfig(True)
    fwd_pipe = fa.HipRotaryGroupedAttention(hip, dtype)
    bq, bk, bv, bdo = (fwd_pipe.upload(x) for x in (q, k, v, do))
    out = fwd_pipe.forward_resident(bq, bk, bv, shape, cfg, None)
    res = fwd_pipe.download_attention(out, shape)
    o = fa.storage_to_f32(res.output, dtype)
    want = oracle.backward_grouped(q, k, v, do, o, res.lse, B, Hq, Hkv, S, D, True, threads=8)
    pipe = fa.HipGroupedBackwardRecomputePipeline(hip, dtype)
    lay = pipe.layout(shape)
    eb = 4 if dtype == fa.DTYPE_F32 else 2
    dq = fa.DeviceBuffer(hip, lay.q_elements * eb)
    dk = fa.DeviceBuffer(hip, lay.kv_elements * eb)
    dv = fa.DeviceBuffer(hip, lay.kv_elements * eb)
    flay = fwd_pipe.layout(shape)
    pipe.encode_tensors(bq, bk, bv, bdo, out, out.ptr + flay.lse_byte_offset, dq, dk, dv, shape,
                        cfg)
    sd = fa.storage_np_dtype(dtype)
    got = [fa.storage_to_f32(b.download(sd, n), dtype)
           for b, n in ((dq, lay.q_elements), (dk, lay.kv_elements), (dv, lay.kv_elements))]
    for name, a, e in zip(("dQ", "dK", "dV"), got, want):
        if dtype == fa.DTYPE_F32:
            assert_close(name, a, e, 5e-4, 2.5e-3)
        else:
            assert_close(name, a, e, 2e-2 * float(np.abs(e).max()), 2e-2)


@pytest.mark.parametrize("causal,scale,dims", [(False, 0.61, (2, 2, 3, 4)), (True, 0.61, (2, 2, 3, 4)),
                                               (True, 0.57, (1, 2, 3, 4))])
def test_m18_canonical_mha_pipeline(hip, causal, scale, dims):
    """tests/m18_wgpu_backward.rs:168 (B2 H2 S3 D4, scale 0.61, both masks) and
    tests/m18_wgpu_backward_pipeline.rs:95 (B1 H2 S3 D4, causal, 0.57), 4e-4 + 2e-3|e|."""
    B, H, S, D = dims
    n = B * H * S * D
    if dims[0] == 2:
        fx = lambda p: _fx(n, p, 0.071, 0.75, 0.1875, 0.43)  # noqa: E731
        q, k, v, do = fx(0.1), fx(0.7), fx(1.3), fx(1.9)
    else:
        fx = lambda p: _fx(n, p, 0.083, 0.625, 0.25, 0.31)  # noqa: E731
        q, k, v, do = fx(0.1), fx(0.7), fx(1.2), fx(1.9)
    o, lse = oracle.forward(q, k, v, B, H, S, D, causal, scale)
    want = oracle.backward_grouped(q, k, v, do, o, lse, B, H, H, S, D, causal, scale)
    shape = fa.AttentionShape(B, H, S, D)
    pipe = fa.HipBackwardRecomputePipeline(hip, fa.DTYPE_F32)
    lay = pipe.layout(shape)
    assert lay.packed_forward_bytes == 4 * (5 * n + B * H * S) and lay.gradient_bytes == 12 * n
    fbuf = fa.DeviceBuffer.from_array(
        hip, fa.pack_backward_recompute_inputs(q, k, v, do, fa.FlatAttentionOutput(o, lse), shape))
    gbuf = pipe.create_gradient_buffer(shape)
    gbuf.fill_u32(0x7FC00000)
    pipe.encode(fbuf, gbuf, shape, fa.FlatAttentionConfig(causal, scale))
    got = [gbuf.download(np.float32, n, off) for off in (0, 4 * n, 8 * n)]
    for name, a, e in zip(("dQ", "dK", "dV"), got, want):
        assert_close(name, a, e, 4e-4, 2e-3)


@pytest.mark.parametrize("dtype", [fa.DTYPE_BF16, fa.DTYPE_F16])
@pytest.mark.parametrize("dims,causal", [((1, 4, 2, 100, 8), True), ((2, 4, 1, 70, 40), False),
                                         ((1, 6, 3, 150, 96), True)])
def test_16bit_partial_head_dims(hip, dtype, dims, causal):
    """Head dims below the padded tile width (32 / 64 / 128 columns): columns >= D are zero in
    every staged tile and never stored."""
    rnd = bf16_round if dtype == fa.DTYPE_BF16 else f16_round
    shape = fa.GroupedAttentionShape(*dims)
    B, Hq, Hkv, S, D = dims
    q, k, v, do = (rnd(normal(n, 51 + i)) for i, n in enumerate(
        (B * Hq * S * D, B * Hkv * S * D, B * Hkv * S * D, B * Hq * S * D)))
    fwd, _ = _expected(q, k, v, do, shape, causal, None)
    fwd = fa.FlatAttentionOutput(rnd(fwd.output), fwd.lse)
    want = oracle.backward_grouped(q, k, v, do, fwd.output, fwd.lse, B, Hq, Hkv, S, D, causal,
                                   threads=8)
    got = fa.HipGroupedBackwardRecomputePipeline(hip, dtype).backward(
        q, k, v, do, fwd, shape, fa.FlatAttentionConfig(causal))
    for name, a, e in zip(("dQ", "dK", "dV"), (got.dq, got.dk, got.dv), want):
        assert_close(name, a, e, 2e-2 * float(np.abs(e).max()), 2e-2)


@pytest.mark.parametrize("dtype", [fa.DTYPE_BF16, fa.DTYPE_F32])
def test_unaligned_tensors_take_the_staged_path(hip, dtype):
    """Tensors at 2-byte (16-bit) / 4-byte (f32) offsets: no 16-byte loads or buffer->LDS
    transfers are possible, the kernels stage through registers (telemetry names the reason);
    results equal the aligned call's bit for bit."""
    B, Hq, Hkv, S, D = 1, 4, 2, 130, 64
    rnd = bf16_round if dtype == fa.DTYPE_BF16 else (lambda x: x)
    q, k, v, do = (rnd(normal(n, 61 + i)) for i, n in enumerate(
        (B * Hq * S * D, B * Hkv * S * D, B * Hkv * S * D, B * Hq * S * D)))
    shape = fa.GroupedAttentionShape(B, Hq, Hkv, S, D)
    fwd, _ = _expected(q, k, v, do, shape, True, None)
    o = rnd(fwd.output)
    eb = 2 if dtype == fa.DTYPE_BF16 else 4
    pipe = fa.HipGroupedBackwardRecomputePipeline(hip, dtype)
    lay = pipe.layout(shape)
    cfg = fa.FlatAttentionConfig(True)

    def run(shift):
        ins = [fa.host_storage(x, dtype) for x in (q, k, v, do, o)] + [fwd.lse.astype(np.float32)]
        bufs = []
        for x in ins:
            b = fa.DeviceBuffer(hip, x.nbytes + 64)
            b.upload(x, shift)
            bufs.append(b)
        outs = [fa.DeviceBuffer(hip, n * eb + 64) for n in (lay.q_elements, lay.kv_elements,
                                                          lay.kv_elements)]
        view = lambda b: fa.DeviceBuffer(hip, b.nbytes - shift, b.ptr + shift)  # noqa: E731
        pipe.encode_tensors(*(view(b) for b in bufs[:5]), bufs[5].ptr + shift,
                            *(view(b) for b in outs), shape, cfg)
        tele = hip.last_telemetry()
        res = [b.download(np.uint8, n * eb, shift) for b, n in zip(
            outs, (lay.q_elements, lay.kv_elements, lay.kv_elements))]
        for b in bufs + outs:
            b.free()
        return res, tele

    aligned, t0 = run(0)
    shifted, t1 = run(eb)
    assert t0.fallback_reason is None and t1.fallback_reason is not None
    for a, b_ in zip(aligned, shifted):
        np.testing.assert_array_equal(a, b_)
    want = oracle.backward_grouped(q, k, v, do, o, fwd.lse, B, Hq, Hkv, S, D, True)
    got = [fa.storage_to_f32(x.view(fa.storage_np_dtype(dtype)), dtype) for x in aligned]
    tol = (5e-4, 2.5e-3) if dtype == fa.DTYPE_F32 else None
    for name, a, e in zip(("dQ", "dK", "dV"), got, want):
        if tol:
            assert_close(name, a, e, *tol)
        else:
            assert_close(name, a, e, 2e-2 * float(np.abs(e).max()), 2e-2)


@pytest.mark.parametrize("dtype", [fa.DTYPE_BF16, fa.DTYPE_F16])
@pytest.mark.parametrize("dims,causal", [((1, 8, 2, 256, 128), True), ((2, 4, 4, 130, 64), False),
                                         ((1, 4, 1, 77, 32), True), ((1, 6, 3, 200, 96), False),
                                         ((1, 2, 1, 33, 128), True)])
def test_stored_ds_path_matches_recompute_path(hip, request, dtype, dims, causal):
    """16-bit storage, aligned tensors: by default bwd_dkdv also writes dS (32 x 32 blocks of the
    storage type) and dQ = dS K reads it back (telemetry names bwd_dq_ds); policy 0 recomputes S
    and dP in bwd_dq. Both use the same dS values in the same MFMA order, so the gradients agree
    bit for bit, and both match the oracle. Ragged lengths leave partial key blocks, whose keys
    past the sequence must read as zero dS."""
    rnd = bf16_round if dtype == fa.DTYPE_BF16 else f16_round
    shape = fa.GroupedAttentionShape(*dims)
    B, Hq, Hkv, S, D = dims
    q, k, v, do = (rnd(normal(n, 71 + i)) for i, n in enumerate(
        (B * Hq * S * D, B * Hkv * S * D, B * Hkv * S * D, B * Hq * S * D)))
    fwd, _ = _expected(q, k, v, do, shape, causal, None)
    fwd = fa.FlatAttentionOutput(rnd(fwd.output), fwd.lse)
    want = oracle.backward_grouped(q, k, v, do, fwd.output, fwd.lse, B, Hq, Hkv, S, D, causal,
                                   threads=8)
    pipe = fa.HipGroupedBackwardRecomputePipeline(hip, dtype)
    request.addfinalizer(lambda: hip.set_backward_policy(-1))
    # the HIP dK/dV kernel on both paths (the assembly one rounds K * scale * log2 e once and is
    # compared with tolerances in test_gpu_backward_assembly.py)
    request.addfinalizer(lambda: hip.set_backward_kernel(-1))
    hip.set_backward_kernel(0)
    runs = {}
    for policy in (-1, 0):
        hip.set_backward_policy(policy)
        got = pipe.backward(q, k, v, do, fwd, shape, fa.FlatAttentionConfig(causal))
        runs[policy] = (got, hip.last_telemetry().kernel_name)
    assert "bwd_dq_ds" in runs[-1][1] and "bwd_dq_ds" not in runs[0][1]
    for name, a, b_, e in zip(("dQ", "dK", "dV"), (runs[-1][0].dq, runs[-1][0].dk, runs[-1][0].dv),
                              (runs[0][0].dq, runs[0][0].dk, runs[0][0].dv), want):
        np.testing.assert_array_equal(a, b_, err_msg=name)
        assert_close(name, a, e, 2e-2 * float(np.abs(e).max()), 2e-2)


def test_stored_ds_falls_back_to_recompute_past_2gib(hip):
    """The dS workspace is used only under 2 GiB: one causal head of 49,152 tokens needs
    2 nt (nt + 1) groups of 8 KiB with nt = 384 (2.42 GB), so the default policy takes the
    recompute path (telemetry names bwd_dq). The long-sequence offsets stay in range: every
    gradient is finite, and dV of the last 64 keys, which only the last 64 queries see, matches
    a float64 evaluation with the forward's own LSE."""
    B, Hq, Hkv, S, D = 1, 1, 1, 49152, 64
    q, k, v, do = (bf16_round(normal(n, 81 + i)) for i, n in enumerate((S * D,) * 4))
    shape = fa.GroupedAttentionShape(B, Hq, Hkv, S, D)
    fwd_pipe = fa.HipRotaryGroupedAttention(hip, fa.DTYPE_BF16)
    res = fwd_pipe.forward(q, k, v, shape, fa.FlatAttentionConfig(True), None)
    o = fa.storage_to_f32(res.output, fa.DTYPE_BF16)
    got = fa.HipGroupedBackwardRecomputePipeline(hip, fa.DTYPE_BF16).backward(
        q, k, v, do, fa.FlatAttentionOutput(o, res.lse), shape, fa.FlatAttentionConfig(True))
    assert "bwd_dq<" in hip.last_telemetry().kernel_name
    for name, x in (("dQ", got.dq), ("dK", got.dk), ("dV", got.dv)):
        assert np.isfinite(x).all(), name
    # dV of key j = sum over queries q >= j of P[q, j] dO[q]: for the last W keys only the last W
    # queries contribute, and P[q, j] = exp(s_qj - LSE_q) uses the full-row LSE the forward gave.
    W = 64
    qs, ks = q.reshape(S, D)[-W:], k.reshape(S, D)[-W:]
    sc = (qs @ ks.T) / np.sqrt(D)
    mask = np.tril(np.ones((W, W), bool))
    p = np.where(mask, np.exp(sc - res.lse[-W:, None]), 0.0)
    dv_want = p.T @ do.reshape(S, D)[-W:]
    assert_close("dV-tail", got.dv.reshape(S, D)[-W:], dv_want,
                 2e-2 * float(np.abs(dv_want).max()), 2e-2)


def fx_m20_adversarial(n, phase):
    """tests/m20_adversarial_numerics.rs:48 fixture: bucketed values up to +-2.09 with
    alternating signs and a small ripple (adversarial but finite)."""
    i = np.arange(n, dtype=np.int64)
    bucket = ((i * 17 + phase * 11) % 23 - 11).astype(np.float32)
    sign = np.where((i + phase) % 2 == 0, 1.0, -1.0).astype(np.float32)
    ripple = np.sin((i + phase).astype(np.float32) * np.float32(0.013)) * np.float32(0.07)
    return (sign * bucket * np.float32(0.19) + ripple).astype(np.float32)


M20_ADVERSARIAL = [((1, 8, 2, 17, 64), True, None), ((1, 8, 1, 33, 32), False, 0.31)]


@pytest.mark.parametrize("idx", range(len(M20_ADVERSARIAL)))
def test_m20_adversarial_numerics(hip, idx):
    """tests/m20_adversarial_numerics.rs:200: the grouped backward on adversarial but finite
    inputs (phases index * 13 + 1, 3, 5, 7 for Q, K, V, dO), 1e-3 + 5e-3 |e|, every gradient
    finite."""
    dims, causal, scale = M20_ADVERSARIAL[idx]
    ph = idx * 13
    _packed_case(hip, fa.GroupedAttentionShape(*dims), fa.FlatAttentionConfig(causal, scale),
                 fx_m20_adversarial, (ph + 1, ph + 3, ph + 5, ph + 7), 1, 1e-3, 5e-3)


@pytest.mark.parametrize("idx", range(len(M20_ADVERSARIAL)))
def test_m20_adversarial_numerics_bf16_stored_ds(hip, idx):
    """The same adversarial inputs rounded to bf16 through the default 16-bit path (dS stored by
    the dK/dV kernel): against the oracle given the same rounded inputs and forward."""
    dims, causal, scale = M20_ADVERSARIAL[idx]
    B, Hq, Hkv, S, D = dims
    ph = idx * 13
    q, k, v, do = (bf16_round(fx_m20_adversarial(n, ph + p)) for n, p in (
        (B * Hq * S * D, 1), (B * Hkv * S * D, 3), (B * Hkv * S * D, 5), (B * Hq * S * D, 7)))
    shape = fa.GroupedAttentionShape(*dims)
    fwd, _ = _expected(q, k, v, do, shape, causal, scale)
    fwd = fa.FlatAttentionOutput(bf16_round(fwd.output), fwd.lse)
    want = oracle.backward_grouped(q, k, v, do, fwd.output, fwd.lse, B, Hq, Hkv, S, D, causal,
                                   scale, threads=8)
    got = fa.HipGroupedBackwardRecomputePipeline(hip, fa.DTYPE_BF16).backward(
        q, k, v, do, fwd, shape, fa.FlatAttentionConfig(causal, scale))
    assert "bwd_dq_ds" in hip.last_telemetry().kernel_name
    for name, a, e in zip(("dQ", "dK", "dV"), (got.dq, got.dk, got.dv), want):
        assert_close(name, a, e, 2e-2 * float(np.abs(e).max()), 2e-2)
