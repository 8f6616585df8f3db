"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the GPU checker.

Each check is chosen so that a plausible restatement mistake (dropped term, wrong sign or index,
transposed operand, wrong RoPE frequency/position, wrong causal offset) fails it:
  * float64 two-pass softmax attention (tests/parity.rs:1-50 naive_forward), tolerance 2e-6;
  * closed forms: Q = 0 -> O = mean of visible V and LSE = ln(#visible); V = 1 -> O = 1;
    causal row 0 -> O = V[0], LSE = scale * q0.k0 (tests/m38_property_stress.rs:79-105);
  * RoPE: position 0 is the identity, pair norms are preserved, the (cos, sin) angle equals
    pos * theta^(-2j/D) evaluated independently in float64, and materialise-then-attend is
    bit-exact to the fused oracle (tests/rotary_grouped.rs:15-135);
  * asymmetric == grouped for equal lengths, decode == last row of the full forward, chunked ==
    contiguous for every chunk size (src/projection_asymmetric.rs:253-347,
    src/chunked_projection_prefill.rs:194-259), bit-exact;
  * paged gather with a shuffled table == contiguous, bit-exact;
  * binary16 / bfloat16 known encodings (src/f16.rs:146-191).
"""
import math

import numpy as np
import pytest

import oracle
from _inputs import Lcg, normal
from conftest import assert_close


def naive64(q, k, v, B, Hq, Hkv, S, D, causal, scale=None, qpos_off=0, kv_len=None,
            layout="bhsd", q_len=None):
    """Two-pass float64 softmax attention (independent of the oracle's loop structure)."""
    q_len = q_len or S
    kv_len = kv_len or S
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    if layout == "bhsd":
        Q = q.reshape(B, Hq, q_len, D).astype(np.float64)
        K = k.reshape(B, Hkv, kv_len, D).astype(np.float64)
        V = v.reshape(B, Hkv, kv_len, D).astype(np.float64)
    else:  # projection [B, S, H*D]
        Q = q.reshape(B, q_len, Hq, D).transpose(0, 2, 1, 3).astype(np.float64)
        K = k.reshape(B, kv_len, Hkv, D).transpose(0, 2, 1, 3).astype(np.float64)
        V = v.reshape(B, kv_len, Hkv, D).transpose(0, 2, 1, 3).astype(np.float64)
    G = Hq // Hkv
    K = np.repeat(K, G, axis=1)
    V = np.repeat(V, G, axis=1)
    s = np.einsum("bhqd,bhkd->bhqk", Q, K) * scale
    if causal:
        qi = np.arange(q_len)[:, None] + qpos_off
        kj = np.arange(kv_len)[None, :]
        s = np.where(kj > qi, -np.inf, s)
    m = s.max(-1, keepdims=True)
    p = np.exp(s - m)
    l = p.sum(-1, keepdims=True)
    o = (p / l) @ V
    lse = (m + np.log(l))[..., 0]
    if layout != "bhsd":
        o = o.transpose(0, 2, 1, 3)
    return o.ravel(), lse.ravel()


def rope64(x, rows, heads, D, theta, positions):
    """Independent float64 RoPE (interleaved pairs), for tolerance checks only."""
    x = x.reshape(rows, heads, D // 2, 2).astype(np.float64)
    j = np.arange(D // 2)
    freq = np.float64(theta) ** (-2.0 * j / D)
    ang = np.asarray(positions, np.float64)[:, None] * freq[None, :]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    e, o = x[..., 0], x[..., 1]
    return np.stack([e * c - o * s, e * s + o * c], -1).reshape(-1)


# --------------------------------------------------------------------------- online softmax


@pytest.mark.parametrize("B,Hq,Hkv,S,D", [(1, 2, 2, 128, 64), (2, 4, 2, 33, 16), (1, 6, 1, 70, 8),
                                          (2, 3, 3, 5, 128)])
@pytest.mark.parametrize("causal", [False, True])
def test_grouped_oracle_matches_float64_two_pass(B, Hq, Hkv, S, D, causal):
    q, k, v = normal(B * Hq * S * D, 1), normal(B * Hkv * S * D, 2), normal(B * Hkv * S * D, 3)
    o, l = oracle.forward_grouped(q, k, v, B, Hq, Hkv, S, D, causal)
    eo, el = naive64(q, k, v, B, Hq, Hkv, S, D, causal)
    assert_close("O", o, eo, 2e-6, 2e-6)
    assert_close("LSE", l, el, 2e-6, 2e-6)


def test_mha_oracle_is_grouped_with_equal_heads():
    B, H, S, D = 2, 3, 40, 32
    q, k, v = normal(B * H * S * D, 4), normal(B * H * S * D, 5), normal(B * H * S * D, 6)
    a = oracle.forward(q, k, v, B, H, S, D, True)
    b = oracle.forward_grouped(q, k, v, B, H, H, S, D, True)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_explicit_scale_is_used():
    B, H, S, D = 1, 1, 9, 4
    q, k, v = normal(B * H * S * D, 1), normal(B * H * S * D, 2), normal(B * H * S * D, 3)
    o, l = oracle.forward(q, k, v, B, H, S, D, False, scale=0.7)
    eo, el = naive64(q, k, v, B, H, H, S, D, False, scale=0.7)
    assert_close("O", o, eo, 2e-6, 2e-6)
    assert_close("LSE", l, el, 2e-6, 2e-6)


def test_closed_forms():
    B, H, S, D = 1, 2, 20, 16
    k, v = normal(B * H * S * D, 7), normal(B * H * S * D, 8)
    zeros = np.zeros(B * H * S * D, np.float32)
    for causal in (False, True):
        o, l = oracle.forward(zeros, k, v, B, H, S, D, causal)
        V = v.reshape(B, H, S, D).astype(np.float64)
        n = np.arange(1, S + 1) if causal else np.full(S, S)
        mean = (np.cumsum(V, axis=2) / n[None, None, :, None]) if causal else \
            np.broadcast_to(V.mean(axis=2, keepdims=True), V.shape)
        assert_close("Q=0 O", o, mean.ravel(), 1e-6, 1e-6)
        assert_close("Q=0 LSE", l, np.tile(np.log(n), B * H), 1e-6, 0)
    q = normal(B * H * S * D, 9)
    o, _ = oracle.forward(q, k, np.ones_like(v), B, H, S, D, True)
    assert np.max(np.abs(o - 1)) <= 3e-6
    o, l = oracle.forward(q, k, v, B, H, S, D, True)
    for h in range(H):
        base = h * S * D
        assert np.array_equal(o[base:base + D], v[base:base + D])
        dot = np.float32(0)
        for d in range(D):
            dot = np.float32(dot + np.float32(q[base + d] * k[base + d]))
        assert l[h * S] == np.float32(dot * np.float32(1 / math.sqrt(D)))


def test_m38_property_stress_lcg_cases():
    """tests/m38_property_stress.rs:45: 64 random cases; V = 1 -> O = 1 (3e-5); causal row 0
    equals V[0] within 2e-4 + 1e-3|e|."""
    rng = Lcg()
    for case in range(64):
        batch = 1 + rng.pick(2)
        hq = [1, 2, 4, 8][rng.pick(4)]
        divs = [c for c in range(1, hq + 1) if hq % c == 0]
        hkv = divs[rng.pick(len(divs))]
        S = 1 + rng.pick(33)
        D = [1, 2, 4, 8, 16, 32, 64, 128][rng.pick(8)]
        q = rng.vec(batch * hq * S * D)
        k = rng.vec(batch * hkv * S * D)
        v = rng.vec(batch * hkv * S * D)
        causal = case % 2 == 0
        o, l = oracle.forward_grouped(q, k, v, batch, hq, hkv, S, D, causal)
        assert np.all(np.isfinite(o)) and np.all(np.isfinite(l))
        o1, _ = oracle.forward_grouped(q, k, np.ones_like(v), batch, hq, hkv, S, D, causal)
        assert np.max(np.abs(o1 - 1)) <= 3e-5, case
        if causal:
            G = hq // hkv
            for b in range(batch):
                for h in range(hq):
                    ob = (b * hq + h) * S * D
                    vb = (b * hkv + h // G) * S * D
                    assert_close("row0", o[ob:ob + D], v[vb:vb + D], 2e-4, 1e-3)


def _policy_fixture(n, kind):
    i = np.arange(n, dtype=np.float32)
    if kind == 0:
        return np.zeros(n, np.float32), np.ones(n, np.float32), (i % 17) * np.float32(0.125) - 1
    if kind == 1:
        return (np.sin(i * np.float32(1e-5)) * np.float32(1e-2)).astype(np.float32), \
               (np.cos(i * np.float32(1e-5)) * np.float32(1e-2)).astype(np.float32), \
               np.sin(i * np.float32(0.031)).astype(np.float32)
    if kind == 2:
        return np.where(np.arange(n) % 2 == 0, 7.75, -7.75).astype(np.float32), \
               np.where((np.arange(n) // 3) % 2 == 0, -6.5, 6.5).astype(np.float32), \
               np.where((np.arange(n) // 5) % 2 == 0, 3.0, -3.0).astype(np.float32)
    return np.where(np.arange(n) % 2 == 0, 24.0, -24.0).astype(np.float32), \
        np.where((np.arange(n) // 2) % 2 == 0, 22.0, -22.0).astype(np.float32), \
        (np.cos(i * np.float32(0.017)) * 4).astype(np.float32)


@pytest.mark.parametrize("kind", range(4))
def test_numerical_policy_corpus_finite_repeatable_and_exact(kind):
    """tests/numerical_policy.rs:12-70: ties, near ties, +-7.75 cancellation, +-24 scores."""
    B, H, S, D = 1, 2, 24, 16
    q, k, v = _policy_fixture(B * H * S * D, kind)
    for causal in (False, True):
        a = oracle.forward(q, k, v, B, H, S, D, causal)
        b = oracle.forward(q, k, v, B, H, S, D, causal)
        assert np.all(np.isfinite(a[0])) and np.all(np.isfinite(a[1]))
        assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
        eo, el = naive64(q, k, v, B, H, H, S, D, causal)
        assert_close("O", a[0], eo, 2e-5, 1e-5)
        assert_close("LSE", a[1], el, 2e-5, 1e-5)


def test_oracle_units_and_threads_agree():
    B, Hq, Hkv, S, D = 2, 4, 2, 30, 32
    q, k, v = normal(B * Hq * S * D, 1), normal(B * Hkv * S * D, 2), normal(B * Hkv * S * D, 3)
    full = oracle.forward_grouped_rope(q, k, v, B, Hq, Hkv, S, D, True, 1e4)
    thr = oracle.forward_grouped_rope(q, k, v, B, Hq, Hkv, S, D, True, 1e4, threads=4)
    assert np.array_equal(full[0], thr[0]) and np.array_equal(full[1], thr[1])
    part = oracle.forward_grouped_rope(q, k, v, B, Hq, Hkv, S, D, True, 1e4, units=(3, 5))
    sl = slice(3 * S * D, 5 * S * D)
    assert np.array_equal(part[0][sl], full[0][sl])


# --------------------------------------------------------------------------- RoPE


def test_rope_identity_at_position_zero_and_norm_preservation():
    D, H = 64, 3
    x = normal(H * D, 1)
    r0 = oracle.rope_rotate_rows(x, 1, H, D, 1e4, 0)
    assert np.array_equal(r0, x)
    r = oracle.rope_rotate_rows(np.tile(x, 50), 50, H, D, 1e4, 7)
    n0 = np.hypot(x[0::2], x[1::2])
    for row in range(50):
        y = r[row * H * D:(row + 1) * H * D]
        assert_close("pair norms", np.hypot(y[0::2], y[1::2]), n0, 1e-6, 1e-6)


@pytest.mark.parametrize("theta", [1e4, 5e5])
def test_rope_matches_float64_frequencies(theta):
    D, rows = 128, 300
    x = normal(rows * D, 2)
    pos = np.arange(rows) * 13 + 5
    r = oracle.rope_rotate_rows(x, rows, 1, D, theta, positions=pos)
    # f32 angle rounding: |angle| <= 4000 rad -> absolute angle error ~ 2.4e-4
    assert_close("rope", r, rope64(x, rows, 1, D, theta, pos), 2e-3, 0)
    # swapping the pair roles (sign error) or using exponent -j/D must fail the same check
    bad = rope64(x, rows, 1, D, theta ** 0.5, pos)
    assert np.max(np.abs(r - bad)) > 1e-1


@pytest.mark.parametrize("hq,hkv", [(4, 4), (8, 2), (4, 1)])
@pytest.mark.parametrize("theta,offset", [(1e4, 0), (5e5, 37)])
@pytest.mark.parametrize("causal", [False, True])
def test_fused_rope_is_bit_exact_to_materialised_rope(hq, hkv, theta, offset, causal):
    """tests/rotary_grouped.rs:49."""
    B, S, D = 2, 19, 16
    q, k, v = normal(B * hq * S * D, 1), normal(B * hkv * S * D, 2), normal(B * hkv * S * D, 3)
    fused = oracle.forward_grouped_rope(q, k, v, B, hq, hkv, S, D, causal, theta, offset)
    qr = oracle.rope_rotate_rows(q, B * hq * S, 1, D, theta,
                                 positions=offset + np.tile(np.arange(S), B * hq))
    kr = oracle.rope_rotate_rows(k, B * hkv * S, 1, D, theta,
                                 positions=offset + np.tile(np.arange(S), B * hkv))
    mat = oracle.forward_grouped(qr, kr, v, B, hq, hkv, S, D, causal)
    assert np.array_equal(fused[0], mat[0]) and np.array_equal(fused[1], mat[1])


def test_fused_rope_matches_float64():
    B, hq, hkv, S, D, theta = 1, 4, 2, 50, 32, 1e4
    q, k, v = normal(B * hq * S * D, 1), normal(B * hkv * S * D, 2), normal(B * hkv * S * D, 3)
    o, l = oracle.forward_grouped_rope(q, k, v, B, hq, hkv, S, D, True, theta, 3)
    pos_q = 3 + np.tile(np.arange(S), B * hq)
    pos_k = 3 + np.tile(np.arange(S), B * hkv)
    qr = rope64(q, B * hq * S, 1, D, theta, pos_q).astype(np.float32)
    kr = rope64(k, B * hkv * S, 1, D, theta, pos_k).astype(np.float32)
    eo, el = naive64(qr, kr, v, B, hq, hkv, S, D, True)
    assert_close("O", o, eo, 1e-5, 1e-5)
    assert_close("LSE", l, el, 1e-5, 1e-5)


# --------------------------------------------------------------------------- asymmetric


def test_asymmetric_equal_length_is_bit_exact_to_grouped_rope():
    """src/projection_asymmetric.rs:253: projection layout with equal lengths == R2."""
    B, hq, hkv, S, D, theta, off = 2, 4, 2, 21, 16, 1e4, 9
    qp, kp, vp = normal(B * S * hq * D, 1), normal(B * S * hkv * D, 2), normal(B * S * hkv * D, 3)
    a = oracle.forward_projection_asymmetric(qp, kp, vp, B, hq, hkv, S, S, D, 0, True, theta,
                                             off, off, True)
    to_bhsd = lambda x, H: x.reshape(B, S, H, D).transpose(0, 2, 1, 3).ravel()  # noqa: E731
    g = oracle.forward_grouped_rope(to_bhsd(qp, hq), to_bhsd(kp, hkv), to_bhsd(vp, hkv), B, hq,
                                    hkv, S, D, True, theta, off)
    assert np.array_equal(a[0], g[0].reshape(B, hq, S, D).transpose(0, 2, 1, 3).ravel())
    assert np.array_equal(a[1], g[1])


def test_decode_is_bit_exact_to_last_row_of_full_forward():
    """src/projection_asymmetric.rs:300-347."""
    hq, hkv, S, D, theta = 4, 2, 25, 16, 1e4
    qp, kp, vp = normal(S * hq * D, 1), normal(S * hkv * D, 2), normal(S * hkv * D, 3)
    full = oracle.forward_projection_asymmetric(qp, kp, vp, 1, hq, hkv, S, S, D, 0, True, theta,
                                                0, 0, True)
    last = qp[(S - 1) * hq * D:]
    dec = oracle.forward_projection_asymmetric(last, kp, vp, 1, hq, hkv, 1, S, D, S - 1, True,
                                               theta, S - 1, 0, True)
    assert np.array_equal(dec[0], full[0][(S - 1) * hq * D:])
    assert np.array_equal(dec[1], full[1].reshape(hq, S)[:, S - 1])


def test_asymmetric_matches_float64_with_offsets():
    B, hq, hkv, ql, kl, D, off = 2, 4, 2, 7, 30, 16, 20
    qp, kp, vp = normal(B * ql * hq * D, 1), normal(B * kl * hkv * D, 2), normal(B * kl * hkv * D, 3)
    o, l = oracle.forward_projection_asymmetric(qp, kp, vp, B, hq, hkv, ql, kl, D, off, True)
    eo, el = naive64(qp, kp, vp, B, hq, hkv, kl, D, True, qpos_off=off, kv_len=kl,
                     layout="proj", q_len=ql)
    assert_close("O", o, eo, 2e-6, 2e-6)
    assert_close("LSE", l, el, 2e-6, 2e-6)


def test_materialised_rope_is_bit_exact_for_asymmetric():
    B, hq, hkv, ql, kl, D, theta = 1, 4, 2, 9, 40, 32, 1e4
    qp, kp, vp = normal(B * ql * hq * D, 1), normal(B * kl * hkv * D, 2), normal(B * kl * hkv * D, 3)
    fused = oracle.forward_projection_asymmetric(qp, kp, vp, B, hq, hkv, ql, kl, D, 31, True,
                                                 theta, 31, 0, True)
    qr = oracle.rope_rotate_rows(qp, ql, hq, D, theta, 31)
    kr = oracle.rope_rotate_rows(kp, kl, hkv, D, theta, 0)
    pre_k = oracle.forward_projection_asymmetric(qp, kr, vp, B, hq, hkv, ql, kl, D, 31, True,
                                                 theta, 31, 0, False)
    none = oracle.forward_projection_asymmetric(qr, kr, vp, B, hq, hkv, ql, kl, D, 31, True, None)
    for other in (pre_k, none):
        assert np.array_equal(fused[0], other[0]) and np.array_equal(fused[1], other[1])


@pytest.mark.parametrize("hq,hkv", [(4, 2), (4, 1)])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("chunk", [1, 2, 3, 4, 8, 16, 100])
def test_chunked_prefill_is_bit_exact_to_contiguous(hq, hkv, causal, chunk):
    """src/chunked_projection_prefill.rs:216-258."""
    B, S, D, theta, off = 2, 13, 16, 1e4, 4
    qp, kp, vp = normal(B * S * hq * D, 1), normal(B * S * hkv * D, 2), normal(B * S * hkv * D, 3)
    c = oracle.chunked_prefill(qp, kp, vp, B, hq, hkv, S, D, causal, theta, off, chunk)
    full = oracle.forward_projection_asymmetric(qp, kp, vp, B, hq, hkv, S, S, D, 0, causal,
                                                theta, off, off, True)
    assert np.array_equal(c[0], full[0]) and np.array_equal(c[1], full[1])


def test_chunked_rejects_zero_chunk():
    x = np.zeros(16, np.float32)
    with pytest.raises(oracle.OracleError) as e:
        oracle.chunked_prefill(x, x, x, 1, 1, 1, 2, 8, True, 1e4, 0, 0)
    assert e.value.code == 28


# --------------------------------------------------------------------------- paged


def test_paged_decode_shuffled_table_is_bit_exact_to_contiguous():
    rng = np.random.default_rng(0)
    hq, hkv, D, ps = 4, 2, 16, 3
    lens = np.array([7, 1, 11], np.int32)
    width = hkv * D
    pages = (lens + ps - 1) // ps
    total = int(pages.sum()) + 2
    perm = rng.permutation(total).astype(np.int32)
    kp = normal(total * ps * width, 1)
    vp = normal(total * ps * width, 2)
    bt = np.zeros((3, pages.max()), np.int32)
    cur = 0
    for s in range(3):
        bt[s, :pages[s]] = perm[cur:cur + pages[s]]
        cur += pages[s]
    q = normal(3 * hq * D, 3)
    o, l = oracle.paged_decode(q, kp, vp, total, ps, bt, lens, hq, hkv, D, True, 1e4)
    for s in range(3):
        rows = [bt[s, t // ps] * ps + t % ps for t in range(lens[s])]
        kc = np.concatenate([kp[r * width:(r + 1) * width] for r in rows])
        vc = np.concatenate([vp[r * width:(r + 1) * width] for r in rows])
        eo, el = oracle.forward_projection_asymmetric(q[s * hq * D:(s + 1) * hq * D], kc, vc, 1, hq,
                                                      hkv, 1, lens[s], D, lens[s] - 1, True, 1e4,
                                                      lens[s] - 1, 0, False)
        assert np.array_equal(o[s * hq * D:(s + 1) * hq * D], eo)
        assert np.array_equal(l[s * hq:(s + 1) * hq], el)


def test_paged_decode_rejects_bad_pages():
    x = np.zeros(64, np.float32)
    with pytest.raises(oracle.OracleError) as e:
        oracle.paged_decode(x[:8], x, x, 2, 4, np.array([[0, 9]], np.int32), [6], 1, 1, 8,
                            True, 1e4)
    assert e.value.code == 30


def test_split_k_lse_combine_closed_form():
    """m = max m_i, l = sum l_i e^{m_i-m}, O = sum O_i l_i e^{m_i-m} / l reproduces the
    unsplit softmax (the merge the GPU decode combine performs)."""
    rng = np.random.default_rng(1)
    s = rng.standard_normal(1000) * 3
    v = rng.standard_normal((1000, 8))
    full_m = s.max()
    p = np.exp(s - full_m)
    full_o = (p[:, None] * v).sum(0) / p.sum()
    full_lse = full_m + np.log(p.sum())
    parts = np.split(np.arange(1000), [17, 300, 301, 999])
    ms, ls, os_ = [], [], []
    for idx in parts:
        m = s[idx].max()
        e = np.exp(s[idx] - m)
        ms.append(m)
        ls.append(e.sum())
        os_.append((e[:, None] * v[idx]).sum(0) / e.sum())
    M = max(ms)
    L = sum(li * np.exp(mi - M) for mi, li in zip(ms, ls))
    O = sum(oi * li * np.exp(mi - M) for oi, li, mi in zip(os_, ls, ms)) / L
    assert np.allclose(O, full_o, atol=1e-12) and abs(M + np.log(L) - full_lse) < 1e-12


# --------------------------------------------------------------------------- 16-bit codecs


def test_binary16_known_encodings():
    """src/f16.rs:150-166."""
    enc = oracle.f32_to_f16(np.array([0.0, -0.0, 1.0, -2.0, 65504.0, np.inf], np.float32))
    assert enc.tolist() == [0x0000, 0x8000, 0x3C00, 0xC000, 0x7BFF, 0x7C00]
    dec = oracle.f16_to_f32(np.array([0x3C00, 0xC000, 0x0400, 0x0001], np.uint16))
    assert dec.tolist() == [1.0, -2.0, 2.0 ** -14, 2.0 ** -24]
    vals = np.array([-17.75, -1.0, -0.33325, 0.0, 0.1, 1.0, np.pi, 1024.5], np.float32)
    rt = oracle.f16_to_f32(oracle.f32_to_f16(vals))
    assert np.all(np.abs(rt - vals) <= 5e-4 * np.maximum(np.abs(vals), 1))
    # agrees with numpy's IEEE binary16 (round-to-nearest-even) on random values
    x = normal(100000, 5) * np.float32(300)
    assert np.array_equal(oracle.f32_to_f16(x), x.astype(np.float16).view(np.uint16))


def test_bfloat16_round_to_nearest_even():
    cases = {1.0: 0x3F80, -2.0: 0xC000, 0.0: 0x0000, np.inf: 0x7F80}
    enc = oracle.f32_to_bf16(np.array(list(cases), np.float32))
    assert enc.tolist() == list(cases.values())
    # ties: 1 + 2^-8 is exactly halfway between 1.0 and 1 + 2^-7 -> even (1.0);
    # 1 + 3*2^-8 is halfway between 1+2^-7 and 1+2^-6 -> even (1 + 2^-6)
    ties = np.array([1 + 2 ** -8, 1 + 3 * 2 ** -8], np.float32)
    assert oracle.f32_to_bf16(ties).tolist() == [0x3F80, 0x3F82]
    assert np.isnan(oracle.bf16_to_f32(oracle.f32_to_bf16(np.array([np.nan], np.float32))))[0]
    x = normal(10000, 3)
    rt = oracle.bf16_to_f32(oracle.f32_to_bf16(x))
    assert np.all(np.abs(rt - x) <= np.abs(x) * 2 ** -8)


def test_input_generator_is_standard_normal_and_seeded():
    x = normal(200000, 77)
    assert abs(float(x.mean())) < 0.01 and abs(float(x.std()) - 1) < 0.01
    assert np.array_equal(x, normal(200000, 77)) and not np.array_equal(x, normal(200000, 78))


def _paged_prefill_case(seed, n, ps, kv_len, hq, hkv, D, shuffled):
    """Pool of pages for n sequences of kv_len rows; identity or shuffled physical ids, plus two
    spare pages that no table names (filled with sentinels that would show in any wrong gather)."""
    rng = np.random.default_rng(seed)
    width = hkv * D
    pages = (kv_len + ps - 1) // ps
    total = n * pages + 2
    ids = rng.permutation(total) if shuffled else np.arange(total)
    bt = ids[:n * pages].reshape(n, pages).astype(np.int32)
    kc = normal(n * kv_len * width, 100 + seed)  # logical rows, contiguous per sequence
    vc = normal(n * kv_len * width, 200 + seed)
    kp = np.full(total * ps * width, 17.0, np.float32)
    vp = np.full(total * ps * width, -19.0, np.float32)
    for s in range(n):
        for t in range(kv_len):
            r = (bt[s, t // ps] * ps + t % ps) * width
            kp[r:r + width] = kc[(s * kv_len + t) * width:(s * kv_len + t + 1) * width]
            vp[r:r + width] = vc[(s * kv_len + t) * width:(s * kv_len + t + 1) * width]
    return total, bt, kp, vp, kc, vc


@pytest.mark.parametrize("ps,kv_len,qlen,qoff,causal", [
    (4, 13, 5, 8, True), (16, 40, 8, 32, True), (5, 23, 23, 0, True), (3, 10, 4, 2, False)])
def test_paged_prefill_is_gather_then_asymmetric_bit_exact(ps, kv_len, qlen, qoff, causal):
    """ora_paged_prefill == (gather rows by block table -> forward_projection_asymmetric with
    pre-rotated K) per sequence, bit for bit, and a shuffled table gives the same bits as the
    identity table (src/chunked_projection_prefill.rs:194-259, src/paged_kv.rs:200-270)."""
    n, hq, hkv, D, theta, qro = 3, 4, 2, 8, 1e4, qoff + 3
    q = normal(n * qlen * hq * D, 7)
    results = []
    for shuffled in (False, True):
        total, bt, kp, vp, kc, vc = _paged_prefill_case(1, n, ps, kv_len, hq, hkv, D, shuffled)
        o, l = oracle.paged_prefill(q, kp, vp, total, ps, bt, hq, hkv, qlen, kv_len, D, qoff,
                                    causal, theta, qro)
        qw, kw = qlen * hq * D, kv_len * hkv * D
        for s in range(n):
            eo, el = oracle.forward_projection_asymmetric(
                q[s * qw:(s + 1) * qw], kc[s * kw:(s + 1) * kw], vc[s * kw:(s + 1) * kw], 1, hq,
                hkv, qlen, kv_len, D, qoff, causal, theta, qro, 0, False)
            assert np.array_equal(o[s * qw:(s + 1) * qw], eo)
            assert np.array_equal(l[s * hq * qlen:(s + 1) * hq * qlen], el)
        results.append((o, l))
    assert np.array_equal(results[0][0], results[1][0])
    assert np.array_equal(results[0][1], results[1][1])
    # Independent float64 check: rotate Q at q_rope_offset, attend over the logical rows.
    o, l = results[1]
    for s in range(n):
        qs = q[s * qlen * hq * D:(s + 1) * qlen * hq * D]
        qr = oracle.rope_rotate_rows(qs, qlen, hq, D, theta, qro)
        eo, el = naive64(qr, kc[s * kv_len * hkv * D:(s + 1) * kv_len * hkv * D],
                         vc[s * kv_len * hkv * D:(s + 1) * kv_len * hkv * D], 1, hq, hkv, None, D,
                         causal, qpos_off=qoff, kv_len=kv_len, layout="proj", q_len=qlen)
        assert_close("paged O", o[s * qlen * hq * D:(s + 1) * qlen * hq * D], eo, 2e-5, 1e-4)
        assert_close("paged LSE", l[s * hq * qlen:(s + 1) * hq * qlen], el, 2e-5, 1e-4)


def test_paged_prefill_rejects_bad_pages_and_short_tables():
    x = np.zeros(4096, np.float32)
    with pytest.raises(oracle.OracleError) as e:  # physical id 9 outside a 2-page pool
        oracle.paged_prefill(x[:16], x, x, 2, 4, np.array([[0, 9]], np.int32), 1, 1, 2, 6, 8, 4,
                             True, 1e4, 4)
    assert e.value.code == 30
    with pytest.raises(oracle.OracleError):  # 6 rows need 2 pages, the table holds 1
        oracle.paged_prefill(x[:16], x, x, 2, 4, np.array([[0]], np.int32), 1, 1, 2, 6, 8, 4,
                             True, 1e4, 4)


def _fx37(n, phase):  # tests/grouped.rs:5
    x = np.arange(n, dtype=np.float32) * np.float32(0.037) + np.float32(phase)
    return (np.sin(x) * np.float32(1.75) + np.cos(x * np.float32(0.41)) * np.float32(0.25)).astype(
        np.float32)


@pytest.mark.parametrize("hq,hkv", [(8, 8), (8, 2), (8, 1)])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("scale", [None, 0.19])
def test_grouped_oracle_matches_expanded_mha_oracle_bit_exactly(hq, hkv, causal, scale):
    """grouped_oracle_matches_expanded_mha_oracle_bit_exactly tests/grouped.rs:30: B2 S7 D16;
    K/V copied out to every query head of their group give the same bits through the MHA oracle
    (and MQA storage is never expanded by the grouped one)."""
    B, S, D = 2, 7, 16
    q = _fx37(B * hq * S * D, 0.1)
    k = _fx37(B * hkv * S * D, 0.7)
    v = _fx37(B * hkv * S * D, 1.3)
    g = oracle.forward_grouped(q, k, v, B, hq, hkv, S, D, causal, scale=scale)
    expand = lambda x: np.repeat(x.reshape(B, hkv, S * D), hq // hkv, axis=1).ravel()  # noqa: E731
    m = oracle.forward(q, expand(k), expand(v), B, hq, S, D, causal, scale=scale)
    assert np.array_equal(g[0].view(np.uint32), m[0].view(np.uint32))
    assert np.array_equal(g[1].view(np.uint32), m[1].view(np.uint32))


@pytest.mark.parametrize("dims", [(1, 4, 4, 7, 16), (2, 8, 2, 9, 64), (1, 8, 1, 5, 32)])
@pytest.mark.parametrize("theta,off", [(1e4, 0), (5e5, 19)])
@pytest.mark.parametrize("causal", [False, True])
def test_projection_oracle_is_bit_exact_with_canonical_after_layout_transform(dims, theta, off,
                                                                              causal):
    """projection_oracle_is_bit_exact_with_canonical_r1_after_layout_transform
    tests/projection_grouped.rs:73: the projection-layout RoPE oracle equals the head-major one
    after moving [B, S, H*D] to [B, H, S, D], bit for bit."""
    B, hq, hkv, S, D = dims
    qp = _fx37(B * S * hq * D, 0.3)
    kp = _fx37(B * S * hkv * D, 0.9)
    vp = _fx37(B * S * hkv * D, 1.5)
    a = oracle.forward_projection_asymmetric(qp, kp, vp, B, hq, hkv, S, S, D, 0, causal, theta,
                                             off, off, True)
    to_bhsd = lambda x, H: x.reshape(B, S, H, D).transpose(0, 2, 1, 3).ravel()  # noqa: E731
    g = oracle.forward_grouped_rope(to_bhsd(qp, hq), to_bhsd(kp, hkv), to_bhsd(vp, hkv), B, hq,
                                    hkv, S, D, causal, theta, off)
    assert np.array_equal(a[0].view(np.uint32),
                          g[0].reshape(B, hq, S, D).transpose(0, 2, 1, 3).ravel().view(np.uint32))
    assert np.array_equal(a[1].view(np.uint32), g[1].view(np.uint32))
