"""GPU parity of the assembly dK/dV backward kernels (fa_bwd_dkdv_a64_bf16 and its f16 twin
fa_bwd_dkdv_a64_f16, generated gfx950 code,
selected by fa_ctx_set_backward_kernel) against the CPU oracle (backward_reference_grouped,
src/backward_grouped.rs:17) and against the HIP dK/dV kernel on the same inputs.

The kernel folds -LSE / scale and -delta into the MFMA accumulator inputs of S and dP (the HIP
kernel subtracts after the products), so the two agree to the bf16 rounding of P and dS, not
bitwise. The bar against the oracle is the 16-bit storage one of the other backward tests:
2e-2 of the tensor's largest magnitude plus 2e-2 |e|; against the HIP kernel 1e-2 of the
largest magnitude (the same products, rounded at different points)."""
import numpy as np
import pytest

import oracle
from _inputs import bf16_round, f16_round, normal
from conftest import assert_close

import flat_attention_amd as fa

pytestmark = pytest.mark.gpu


def _inputs(dims, seed, rnd=bf16_round, amp=1.0):
    B, Hq, Hkv, S, D = dims
    return tuple(rnd(np.float32(amp) * normal(n, seed + i)) for i, n in enumerate(
        (B * Hq * S * D, B * Hkv * S * D, B * Hkv * S * D, B * Hq * S * D)))


def _run(hip, dims, causal, seed, scale=None, kernel=-1, dtype=fa.DTYPE_BF16, amp=1.0):
    rnd = bf16_round if dtype == fa.DTYPE_BF16 else f16_round
    B, Hq, Hkv, S, D = dims
    shape = fa.GroupedAttentionShape(*dims)
    q, k, v, do = _inputs(dims, seed, rnd, amp)
    o, lse = oracle.forward_grouped(q, k, v, B, Hq, Hkv, S, D, causal, scale)
    fwd = fa.FlatAttentionOutput(rnd(o), lse)
    want = oracle.backward_grouped(q, k, v, do, fwd.output, fwd.lse, B, Hq, Hkv, S, D, causal,
                                   scale, threads=8)
    hip.set_backward_kernel(kernel)
    try:
        got = fa.HipGroupedBackwardRecomputePipeline(hip, dtype).backward(
            q, k, v, do, fwd, shape, fa.FlatAttentionConfig(causal, scale))
        name = hip.last_telemetry().kernel_name
    finally:
        hip.set_backward_kernel(-1)
    return got, want, name


CASES = [
    ((1, 1, 1, 128, 128), True),      # one key block, one tile: diagonal only
    ((1, 1, 1, 128, 128), False),
    ((1, 4, 1, 256, 128), True),      # MQA group of 4, two tiles per head
    ((2, 8, 2, 384, 128), True),
    ((2, 8, 2, 384, 128), False),
    ((1, 2, 2, 512, 128), True),      # MHA
    ((1, 16, 2, 256, 128), False),    # group of 8
]


@pytest.mark.parametrize("dims,causal", CASES)
def test_matches_oracle(hip, dims, causal):
    got, want, name = _run(hip, dims, causal, 301)
    assert "bwd_dkdv_a64" in name, name
    for tag, a, e in zip(("dQ", "dK", "dV"), (got.dq, got.dk, got.dv), want):
        assert np.isfinite(a).all(), tag
        assert_close(f"{dims}-{causal}-{tag}", a, e, 2e-2 * float(np.abs(e).max()), 2e-2)


@pytest.mark.parametrize("dims,causal", [CASES[0], CASES[3], CASES[4], CASES[6]])
def test_f16_matches_oracle(hip, dims, causal):
    """f16 storage: the f16 twin (f16 MFMAs, dS and dK/dV stored as f16)."""
    got, want, name = _run(hip, dims, causal, 305, dtype=fa.DTYPE_F16)
    assert "bwd_dkdv_a64" in name and "<f16>" in name, name
    for tag, a, e in zip(("dQ", "dK", "dV"), (got.dq, got.dk, got.dv), want):
        assert np.isfinite(a).all(), tag
        assert_close(f"{dims}-{causal}-{tag}", a, e, 2e-2 * float(np.abs(e).max()), 2e-2)


@pytest.mark.parametrize("dtype", [fa.DTYPE_BF16, fa.DTYPE_F16])
@pytest.mark.parametrize("dims,causal", [((2, 8, 2, 384, 128), True),
                                         ((1, 16, 2, 256, 128), False)])
def test_agrees_with_hip_kernel(hip, dims, causal, dtype):
    got, _, name = _run(hip, dims, causal, 311, dtype=dtype)
    ref, _, name0 = _run(hip, dims, causal, 311, kernel=0, dtype=dtype)
    assert "bwd_dkdv_a64" in name and "bwd_dkdv_a64" not in name0, (name, name0)
    for tag, a, b in zip(("dQ", "dK", "dV"), (got.dq, got.dk, got.dv),
                         (ref.dq, ref.dk, ref.dv)):
        scale = float(np.abs(b).max())
        assert_close(f"{tag}", a, b, 1e-2 * scale, 1e-2)


@pytest.mark.parametrize("scale", [0.05, 0.3])
def test_explicit_scale_and_peaked_scores(hip, scale):
    """A non-default softmax scale with inputs of amplitude 3: peaked rows, P near 0 and 1."""
    dims = (1, 4, 2, 256, 128)
    got, want, name = _run(hip, dims, True, 321, scale=scale, amp=3.0)
    assert "bwd_dkdv_a64" in name, name
    for tag, a, e in zip(("dQ", "dK", "dV"), (got.dq, got.dk, got.dv), want):
        assert_close(tag, a, e, 2e-2 * float(np.abs(e).max()), 2e-2)


def test_deterministic(hip):
    dims = (1, 8, 2, 256, 128)
    a, _, _ = _run(hip, dims, True, 331)
    b, _, _ = _run(hip, dims, True, 331)
    for x, y in zip((a.dq, a.dk, a.dv), (b.dq, b.dk, b.dv)):
        np.testing.assert_array_equal(x, y)


@pytest.mark.parametrize("dims,dtype", [((1, 4, 2, 130, 128), fa.DTYPE_BF16),   # ragged
                                        ((1, 4, 2, 256, 64), fa.DTYPE_BF16),    # head_dim 64
                                        ((1, 4, 2, 256, 64), fa.DTYPE_F16)])
def test_other_shapes_take_the_hip_kernel(hip, dims, dtype):
    got, want, name = _run(hip, dims, True, 341, dtype=dtype)
    assert "bwd_dkdv_a64" not in name and "bwd_dkdv" in name, name
    for tag, a, e in zip(("dQ", "dK", "dV"), (got.dq, got.dk, got.dv), want):
        assert_close(tag, a, e, 2e-2 * float(np.abs(e).max()), 2e-2)


def test_recompute_policy_takes_the_hip_kernel(hip, request):
    """Without the stored dS (backward policy 0) the assembly kernel does not apply."""
    request.addfinalizer(lambda: hip.set_backward_policy(-1))
    hip.set_backward_policy(0)
    _, _, name = _run(hip, (1, 4, 2, 256, 128), True, 351)
    assert "bwd_dkdv_a64" not in name and "bwd_dq<" in name, name


def test_bench_shape_units_and_closed_forms(hip):
    """The bench shape (B2 Hq32 Hkv8 N4096 D128 bf16, causal) through the library's own forward
    and the default backward: the oracle on the first and the last (batch, kv head) unit (its 4
    query heads, given the same O and LSE), and over every unit the closed forms the softmax
    fixes: each row of P sums to 1, so sum_k dV[k] = sum over the unit's query rows of dO, and
    each row of dS sums to 0, so sum_k dK[k] = 0."""
    B, Hq, Hkv, S, D = 2, 32, 8, 4096, 128
    G = Hq // Hkv
    shape = fa.GroupedAttentionShape(B, Hq, Hkv, S, D)
    cfg = fa.FlatAttentionConfig(True)
    dt = fa.DTYPE_BF16
    q, k, v, do = (bf16_round(normal(n, 361 + i)) for i, n in enumerate(
        (B * Hq * S * D, B * Hkv * S * D, B * Hkv * S * D, B * Hq * S * D)))
    fwd = fa.HipRotaryGroupedAttention(hip, dt).forward(q, k, v, shape, cfg, None)
    o = fa.storage_to_f32(fwd.output, dt)
    got = fa.HipGroupedBackwardRecomputePipeline(hip, dt).backward(
        q, k, v, do, fa.FlatAttentionOutput(o, fwd.lse), shape, cfg)
    assert "bwd_dkdv_a64" in hip.last_telemetry().kernel_name
    dq, dk, dv = (x.reshape(B, -1, S, D) for x in (got.dq, got.dk, got.dv))
    for x in (dq, dk, dv):
        assert np.isfinite(x).all()
    q4, do4, o4 = (x.reshape(B, Hq, S, D) for x in (q, do, o))
    k4, v4 = (x.reshape(B, Hkv, S, D) for x in (k, v))
    lse = np.asarray(fwd.lse, np.float32).reshape(B, Hq, S)
    for b, h in ((0, 0), (B - 1, Hkv - 1)):
        hs = slice(h * G, (h + 1) * G)
        want = oracle.backward_grouped(q4[b, hs], k4[b, h], v4[b, h], do4[b, hs], o4[b, hs],
                                       lse[b, hs], 1, G, 1, S, D, True, threads=8)
        for name, a, e in zip(("dQ", "dK", "dV"), (dq[b, hs], dk[b, h], dv[b, h]), want):
            assert_close(f"unit {b},{h} {name}", a.ravel(), e, 2e-2 * float(np.abs(e).max()),
                         2e-2)
    # closed forms over every unit (float64 sums of the bf16 gradients)
    sum_dv = dv.astype(np.float64).sum(axis=2)                       # [B, Hkv, D]
    want_dv = do4.astype(np.float64).reshape(B, Hkv, G, S, D).sum(axis=(2, 3))
    assert np.abs(sum_dv - want_dv).max() <= 2e-2 * np.abs(want_dv).max()
    sum_dk = dk.astype(np.float64).sum(axis=2)
    assert np.abs(sum_dk).max() <= 2e-2 * np.abs(dk).sum(axis=2).max()
