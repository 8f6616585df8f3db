"""GPU parity of the assembly prefill main loop (the default where it applies; forced with
fa_ctx_set_prefill_kernel(1): fa_prefill_a64_bf16, generated gfx950 code, 64 query rows per wave, persistent grid) against
the CPU oracle, through the C ABI.

Tolerance: 16-bit I/O max-abs 2e-2 on O and LSE after quantising the oracle's inputs to bf16
(tests/wgpu_f16.rs:68-100 convention), the bar the HIP 16-bit kernels meet. The kernel scales Q
by scale * log2 e before its one rounding to bf16 (after the RoPE rotation, which rounds it
anyway), so its results are not bitwise those of the HIP kernel; both are held to the oracle.
"""
import numpy as np
import pytest

import oracle
from _inputs import bf16_round, f16_round, normal
from conftest import assert_close
from test_gpu_prefill import _oracle_grouped, _rope64, _rope_adversarial_inputs, _run_grouped

import flat_attention_amd as fa

pytestmark = pytest.mark.gpu

H16_ATOL = 2e-2


@pytest.fixture
def asm(hip):
    hip.set_prefill_kernel(1)
    try:
        yield hip
    finally:
        hip.set_prefill_kernel(-1)


def _assert_ran_assembly(hip):
    name = hip.last_telemetry().kernel_name
    assert "prefill_a64" in name, name


@pytest.mark.parametrize("hq,hkv", [(1, 1), (4, 4), (8, 2), (32, 8), (16, 1)])
@pytest.mark.parametrize("S", [1, 63, 200, 300, 1000])
@pytest.mark.parametrize("causal", [True, False])
def test_assembly_prefill_matches_oracle(asm, hq, hkv, S, causal):
    """GQA groups 1..16 (the kernel packs group x rows into one 256-row block), ragged key
    tiles (S not a multiple of 64: zero-filled tail rows masked in the softmax), one-row
    sequences, both masks, a RoPE position offset."""
    B, D = 2, 128
    q = bf16_round(normal(B * hq * S * D, 900 + S + hq))
    k = bf16_round(normal(B * hkv * S * D, 901 + S))
    v = bf16_round(normal(B * hkv * S * D, 902 + S))
    shape = fa.GroupedAttentionShape(B, hq, hkv, S, D)
    rot = fa.RotaryEmbeddingConfig(1e4, 7)
    o, l = _run_grouped(asm, q, k, v, shape, fa.FlatAttentionConfig(causal), rot, fa.DTYPE_BF16)
    _assert_ran_assembly(asm)
    units = (0, B * hq) if S <= 300 else (0, 2)
    eo, el = _oracle_grouped(q, k, v, shape, causal, rot, units=units)
    n = (units[1] - units[0]) * S
    assert_close("O", o[:n * D], eo[:n * D], H16_ATOL, 0.0)
    assert_close("LSE", l[:n], el[:n], H16_ATOL, 0.0)
    assert np.isfinite(o).all() and np.isfinite(l).all()


@pytest.mark.parametrize("hq,hkv,S", [(8, 2, 63), (32, 8, 300), (16, 1, 200), (4, 4, 1000)])
@pytest.mark.parametrize("causal", [True, False])
def test_assembly_prefill_f16_matches_oracle_and_hip(asm, hq, hkv, S, causal):
    """f16 storage (fa_prefill_a64_f16: the same schedule with the f16 MFMA and conversions, the
    fast path's overflow threshold at row sums of 2^15): the oracle at the 16-bit bar, and the
    HIP kernel (fa_ctx_set_prefill_kernel(0)) within it."""
    B, D = 2, 128
    q = f16_round(normal(B * hq * S * D, 980 + S + hq))
    k = f16_round(normal(B * hkv * S * D, 981 + S))
    v = f16_round(normal(B * hkv * S * D, 982 + S))
    shape = fa.GroupedAttentionShape(B, hq, hkv, S, D)
    rot = fa.RotaryEmbeddingConfig(1e4, 7)
    cfg = fa.FlatAttentionConfig(causal)
    o, l = _run_grouped(asm, q, k, v, shape, cfg, rot, fa.DTYPE_F16)
    name = asm.last_telemetry().kernel_name
    assert "prefill_a64<f16>" in name, name
    try:
        asm.set_prefill_kernel(0)
        o0, l0 = _run_grouped(asm, q, k, v, shape, cfg, rot, fa.DTYPE_F16)
        assert "prefill_a64" not in asm.last_telemetry().kernel_name
    finally:
        asm.set_prefill_kernel(-1)
    assert np.isfinite(o).all() and np.isfinite(l).all()
    units = (0, B * hq) if S <= 300 else (0, 2)
    eo, el = _oracle_grouped(q, k, v, shape, causal, rot, units=units)
    n = (units[1] - units[0]) * S
    assert_close("O", o[:n * D], eo[:n * D], H16_ATOL, 0.0)
    assert_close("LSE", l[:n], el[:n], H16_ATOL, 0.0)
    assert_close("O vs HIP", o, o0, H16_ATOL, 0.0)
    assert_close("LSE vs HIP", l, l0, H16_ATOL, 0.0)


def test_assembly_prefill_cfg3_full_size(asm):
    """BASELINE configs[2] (B2 Hq32 Hkv8 N4096 D128 bf16, theta 1e4, causal): the oracle on the
    first and last (batch, head) units, V = 1 giving O = 1 on every row, and the persistent grid
    (fewer workgroups than blocks) covering every block."""
    B, hq, hkv, S, D = 2, 32, 8, 4096, 128
    q = bf16_round(normal(B * hq * S * D, 31))
    k = bf16_round(normal(B * hkv * S * D, 32))
    v = bf16_round(normal(B * hkv * S * D, 33))
    shape = fa.GroupedAttentionShape(B, hq, hkv, S, D)
    rot = fa.RotaryEmbeddingConfig(1e4, 0)
    cfg = fa.FlatAttentionConfig(True)
    o, l = _run_grouped(asm, q, k, v, shape, cfg, rot, fa.DTYPE_BF16)
    _assert_ran_assembly(asm)
    t = asm.last_telemetry()
    assert t.workgroups[0] < B * hkv * (S * (hq // hkv) // 256)
    assert np.isfinite(o).all() and np.isfinite(l).all()
    qr = oracle.rope_rotate_rows(q, B * hq * S, 1, D, 1e4, 0,
                                 positions=np.tile(np.arange(S), B * hq))
    kr = oracle.rope_rotate_rows(k, B * hkv * S, 1, D, 1e4, 0,
                                 positions=np.tile(np.arange(S), B * hkv))
    for unit in (0, B * hq - 1):
        eo, el = oracle.forward_grouped(qr, kr, v, B, hq, hkv, S, D, True, units=(unit, unit + 1))
        sl = slice(unit * S * D, (unit + 1) * S * D)
        assert_close(f"O unit {unit}", o[sl], eo[sl], H16_ATOL, 0.0)
        ls = slice(unit * S, (unit + 1) * S)
        assert_close(f"LSE unit {unit}", l[ls], el[ls], H16_ATOL, 0.0)
    ones = bf16_round(np.ones_like(v))
    o1, l1 = _run_grouped(asm, q, k, ones, shape, cfg, rot, fa.DTYPE_BF16)
    assert np.max(np.abs(o1 - 1.0)) <= 2e-2
    assert np.array_equal(l1.view(np.uint32), l.view(np.uint32))
    # the HIP kernel on the same inputs: the two agree within the same bar
    asm.set_prefill_kernel(0)
    o0, l0 = _run_grouped(asm, q, k, v, shape, cfg, rot, fa.DTYPE_BF16)
    assert "prefill_a64" not in asm.last_telemetry().kernel_name
    assert_close("O vs HIP kernel", o, o0, H16_ATOL, 0.0)
    assert_close("LSE vs HIP kernel", l, l0, H16_ATOL, 0.0)


@pytest.mark.parametrize("dtype,rnd", [(fa.DTYPE_BF16, bf16_round), (fa.DTYPE_F16, f16_round)])
@pytest.mark.parametrize("pattern", ["rising", "falling", "alternating"])
def test_assembly_prefill_adversarial_scores(asm, pattern, dtype, rnd):
    """Scores rising to 60 (every tile moves the row max: the exact rescale path on each tile),
    falling to -60 (the max never moves), or alternating +-24, over 4096 RoPE positions. The
    rounding of rotated Q and K to bf16 bounds the LSE error by max|s| * 2^-7, the bound the HIP
    kernel's default mode is held to; O is held to 2e-2 where the scores stay small."""
    S, D, theta = 4096, 128, 1e4
    q, k = _rope_adversarial_inputs(pattern, S, D, theta, False)
    q, k = rnd(q), rnd(k)
    v = rnd(normal(S * D, 77))
    shape = fa.GroupedAttentionShape(1, 1, 1, S, D)
    rot = fa.RotaryEmbeddingConfig(theta, 0)
    qr = oracle.rope_rotate_rows(q, S, 1, D, theta, 0)
    kr = oracle.rope_rotate_rows(k, S, 1, D, theta, 0)
    eo, el = oracle.forward(qr, kr, v, 1, 1, S, D, True)
    smax = float(np.max(np.abs(np.asarray(qr).reshape(S, D) @ np.asarray(kr).reshape(S, D).T
                               / np.sqrt(D))))
    o, l = _run_grouped(asm, q, k, v, shape, fa.FlatAttentionConfig(True), rot, dtype)
    _assert_ran_assembly(asm)
    assert np.isfinite(o).all() and np.isfinite(l).all()
    assert_close("LSE", l, el, smax * 2.0 ** -7, 0.0)
    # O is a convex combination of V rows: it stays inside V's range on every row
    vr = v.reshape(S, D)
    assert np.all(o.reshape(S, D) <= vr.max(axis=0) + 2e-2)
    assert np.all(o.reshape(S, D) >= vr.min(axis=0) - 2e-2)


@pytest.mark.parametrize("dtype,rnd", [(fa.DTYPE_BF16, bf16_round), (fa.DTYPE_F16, f16_round)])
def test_assembly_prefill_tied_and_jumping_scores(asm, dtype, rnd):
    """Ties (zero keys: every score exactly 0, uniform rows with l = t + 1) held to 2e-2, and
    +-24 jumps between neighbouring keys inside each 64-key tile (the row max moves within a
    tile, P underflows for half the keys) held to the RoPE rounding bound max|s| * 2^-7 on LSE
    and to V's range on O."""
    S, D, H, theta = 300, 128, 2, 1e4
    idx = np.arange(S)
    u = np.full(D, 1.0 / np.sqrt(D))
    v = rnd(normal(H * S * D, 5))
    vr = v.reshape(H, S, D)
    shape = fa.GroupedAttentionShape(1, H, H, S, D)
    rot = fa.RotaryEmbeddingConfig(theta, 0)
    for name, scores in (("ties", np.zeros(S)),
                         ("jumps", np.where(idx % 2 == 0, 24.0, -24.0))):
        q1 = _rope64(np.tile(u, (S, 1)), idx, D, theta, -1.0)
        k1 = _rope64(scores[:, None] * np.sqrt(D) * u[None, :], idx, D, theta, -1.0)
        q = rnd(np.tile(q1.astype(np.float32).ravel(), H))
        k = rnd(np.tile(k1.astype(np.float32).ravel(), H))
        for causal in (True, False):
            o, l = _run_grouped(asm, q, k, v, shape, fa.FlatAttentionConfig(causal), rot, dtype)
            _assert_ran_assembly(asm)
            eo, el = _oracle_grouped(q, k, v, shape, causal, rot)
            if name == "ties":
                assert_close(f"O {name}", o, eo, H16_ATOL, 0.0)
                assert_close(f"LSE {name}", l, el, H16_ATOL, 0.0)
            else:
                assert_close(f"LSE {name}", l, el, 24.0 * 2.0 ** -7 + H16_ATOL, 0.0)
                oo = o.reshape(H, S, D)
                assert np.all(oo <= vr.max(axis=1, keepdims=True) + 2e-2)
                assert np.all(oo >= vr.min(axis=1, keepdims=True) - 2e-2)


def test_assembly_projection_layout_rect_causal_offset(asm):
    """Projection-layout rows (heads interleaved in each token row: strides hq * D) and
    rectangular shapes with a causal offset (q_len < kv_len, the chunked-prefill case), and a
    single query row, through the assembly kernel."""
    B, hq, hkv, D, theta = 2, 8, 2, 128, 1e4
    for ql, kl, off in ((1, 77, 76), (19, 90, 71), (64, 64, 0), (40, 300, 260)):
        q = bf16_round(normal(B * ql * hq * D, ql))
        k, v = bf16_round(normal(B * kl * hkv * D, kl)), bf16_round(normal(B * kl * hkv * D, kl + 1))
        shape = fa.AsymmetricGroupedAttentionShape(B, hq, hkv, ql, kl, D, off)
        rot = fa.AsymmetricRotaryEmbeddingConfig(theta, off + 3, 3)
        for causal in (True, False):
            pipe = fa.HipAsymmetricProjectionPipeline(asm, fa.DTYPE_BF16)
            lay = pipe.layout(shape)
            out = fa.DeviceBuffer(asm, lay.combined_bytes)
            qb, kb, vb = (fa.DeviceBuffer.from_array(asm, fa.host_storage(x, fa.DTYPE_BF16))
                          for x in (q, k, v))
            pipe.encode(qb, kb, vb, out, shape, fa.FlatAttentionConfig(causal), rot)
            res = fa.download_attention(out, lay, fa.DTYPE_BF16)
            eo, el = oracle.forward_projection_asymmetric(q, k, v, B, hq, hkv, ql, kl, D, off,
                                                          causal, theta, off + 3, 3, True)
            assert_close(f"O {ql}x{kl}", fa.storage_to_f32(res.output, fa.DTYPE_BF16), eo,
                         H16_ATOL, 0.0)
            assert_close(f"LSE {ql}x{kl}", res.lse, el, H16_ATOL, 0.0)


@pytest.mark.parametrize("case", ["f16_head_dim_64", "head_dim_64", "no_rope", "group_3",
                                  "precise_group_3"])
def test_assembly_prefill_falls_back_where_it_does_not_apply(asm, case):
    """Inputs outside the assembly kernel's scope run the HIP kernels (the telemetry names
    which) and still match the oracle."""
    B, hq, hkv, S, D = 1, 4, 2, 130, 128
    dtype, rnd, rot = fa.DTYPE_BF16, bf16_round, fa.RotaryEmbeddingConfig(1e4, 0)
    if case == "f16_head_dim_64":
        dtype, rnd, D = fa.DTYPE_F16, f16_round, 64
    elif case == "head_dim_64":
        D = 64
    elif case == "no_rope":
        rot = None
    elif case in ("group_3", "precise_group_3"):
        hq, hkv = 6, 2
    q = rnd(normal(B * hq * S * D, 41))
    k, v = rnd(normal(B * hkv * S * D, 42)), rnd(normal(B * hkv * S * D, 43))
    shape = fa.GroupedAttentionShape(B, hq, hkv, S, D)
    try:
        if case == "precise_group_3":
            asm.set_prefill_precision(1)
        o, l = _run_grouped(asm, q, k, v, shape, fa.FlatAttentionConfig(True), rot, dtype)
    finally:
        asm.set_prefill_precision(0)
    assert "prefill_a64" not in asm.last_telemetry().kernel_name
    eo, el = _oracle_grouped(q, k, v, shape, True, rot)
    assert_close("O", o, eo, H16_ATOL, 0.0)
    assert_close("LSE", l, el, H16_ATOL, 0.0)


@pytest.mark.parametrize("hq,hkv,cached,ql,causal", [(32, 8, 300, 200, True),
                                                     (16, 1, 0, 129, True),
                                                     (8, 8, 1000, 64, False),
                                                     (4, 2, 17, 300, True)])
@pytest.mark.parametrize("dtype,rnd", [(fa.DTYPE_BF16, bf16_round), (fa.DTYPE_F16, f16_round)])
def test_assembly_paged_prefill_matches_paged_oracle(asm, hq, hkv, cached, ql, causal, dtype,
                                                     rnd):
    """The paged assembly kernel (16-row pages): chunked prefill over a shuffled page pool whose
    unnamed rows hold NaN (a wrong page shows), GQA groups 1..16, ragged last pages, causal
    offsets from 0 to 1000; checked against the paged oracle over the device's own pool and
    bitwise against the identity block table."""
    from test_gpu_paged import _paged_prefill
    n_seqs, D, ps, theta = 3, 128, 16, 1e4
    kv_len = cached + ql
    pages_per = -(-kv_len // ps)
    total = n_seqs * pages_per + 5
    rng = np.random.default_rng(kv_len + hq)
    width = hkv * D
    raw_k = rnd(normal(n_seqs * kv_len * width, 41))
    v = rnd(normal(n_seqs * kv_len * width, 42))
    q = rnd(normal(n_seqs * ql * hq * D, 43))
    ident = np.arange(n_seqs * pages_per, dtype=np.int32).reshape(n_seqs, pages_per)
    shuf = rng.permutation(total)[:n_seqs * pages_per].astype(np.int32).reshape(n_seqs, pages_per)
    o1, l1 = _paged_prefill(asm, ident, ps, total, n_seqs, hq, hkv, D, cached, ql, theta, raw_k,
                            v, q, dtype, causal)
    _assert_ran_assembly(asm)
    pools = []
    o2, l2 = _paged_prefill(asm, shuf, ps, total, n_seqs, hq, hkv, D, cached, ql, theta, raw_k,
                            v, q, dtype, causal, pools)
    _assert_ran_assembly(asm)
    assert np.array_equal(o1.view(np.uint32), o2.view(np.uint32))
    assert np.array_equal(l1.view(np.uint32), l2.view(np.uint32))
    po, pl = oracle.paged_prefill(q, pools[0], pools[1], total, ps, shuf, hq, hkv, ql, kv_len, D,
                                  cached, causal, theta, cached, threads=4)
    assert_close("O vs paged oracle", o2, po, H16_ATOL, 0.0)
    assert_close("LSE vs paged oracle", l2, pl, H16_ATOL, 0.0)


@pytest.mark.parametrize("hq,hkv,S", [(8, 2, 200), (4, 4, 63), (16, 1, 300), (32, 8, 1000)])
@pytest.mark.parametrize("causal", [True, False])
def test_precise_assembly_prefill_matches_oracle_and_hip_split(hip, hq, hkv, S, causal):
    """Precision mode 1 on the assembly kernel (fa_prefill_a64_precise_bf16: K and its bf16
    residual from the split rotation pre-pass, Q split in the kernel, three score MFMAs per
    k-step, three 48 KiB stages): the oracle at the 16-bit bar, and the HIP split-score kernel
    (fa_ctx_set_prefill_kernel(0)) within it."""
    B, D = 2, 128
    q = bf16_round(normal(B * hq * S * D, 950 + S + hq))
    k = bf16_round(normal(B * hkv * S * D, 951 + S))
    v = bf16_round(normal(B * hkv * S * D, 952 + S))
    shape = fa.GroupedAttentionShape(B, hq, hkv, S, D)
    rot = fa.RotaryEmbeddingConfig(1e4, 5)
    cfg = fa.FlatAttentionConfig(causal)
    try:
        hip.set_prefill_precision(1)
        o, l = _run_grouped(hip, q, k, v, shape, cfg, rot, fa.DTYPE_BF16)
        name = hip.last_telemetry().kernel_name
        assert "prefill_a64" in name and "split" in name, name
        hip.set_prefill_kernel(0)
        o0, l0 = _run_grouped(hip, q, k, v, shape, cfg, rot, fa.DTYPE_BF16)
        assert "prefill_a64" not in hip.last_telemetry().kernel_name
    finally:
        hip.set_prefill_precision(0)
        hip.set_prefill_kernel(-1)
    assert np.isfinite(o).all() and np.isfinite(l).all()
    units = (0, B * hq) if S <= 300 else (0, 2)
    eo, el = _oracle_grouped(q, k, v, shape, causal, rot, units=units)
    n = (units[1] - units[0]) * S
    assert_close("O", o[:n * D], eo[:n * D], H16_ATOL, 0.0)
    assert_close("LSE", l[:n], el[:n], H16_ATOL, 0.0)
    assert_close("O vs HIP split", o, o0, H16_ATOL, 0.0)
    assert_close("LSE vs HIP split", l, l0, H16_ATOL, 0.0)


@pytest.mark.parametrize("dtype,rnd", [(fa.DTYPE_BF16, bf16_round), (fa.DTYPE_F32, lambda x: x)])
def test_kernel_timing_leaves_results_unchanged(hip, dtype, rnd):
    """With per-kernel timing on, the assembly kernel (bf16) and the f32 kernel record their
    span's events as part of their own dispatch: the output is bitwise the one without timing,
    and the prefill kernel shows one timed dispatch of positive duration."""
    B, hq, hkv, S, D = 1, 8, 2, 300, 128
    q = rnd(normal(B * hq * S * D, 971))
    k, v = rnd(normal(B * hkv * S * D, 972)), rnd(normal(B * hkv * S * D, 973))
    shape = fa.GroupedAttentionShape(B, hq, hkv, S, D)
    cfg, rot = fa.FlatAttentionConfig(True), fa.RotaryEmbeddingConfig(1e4, 0)
    o0, l0 = _run_grouped(hip, q, k, v, shape, cfg, rot, dtype)
    hip.set_kernel_timing(True)
    try:
        o1, l1 = _run_grouped(hip, q, k, v, shape, cfg, rot, dtype)
        t = hip.last_telemetry()
        if dtype == fa.DTYPE_BF16:
            assert "prefill_a64" in t.kernel_name, t.kernel_name
        ms, n = hip.kernel_timing(t.kernel_id)
        assert n == 1 and ms > 0.0, (t.kernel_id, ms, n)
    finally:
        hip.set_kernel_timing(False)
    assert np.array_equal(o0.view(np.uint32), o1.view(np.uint32))
    assert np.array_equal(l0.view(np.uint32), l1.view(np.uint32))
