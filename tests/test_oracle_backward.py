"""Pins the recompute-backward oracle (ora_backward_grouped, following
src/backward_grouped.rs:17-95) before it is trusted as the GPU checker.

Each check is chosen so that a plausible restatement mistake fails it:
  * central finite differences of the objective sum(dO * O) through the (separately pinned)
    forward oracle, with the reference's own fixture, epsilon and tolerance
    (src/backward_grouped.rs:100-212): a dropped delta term, a wrong sign or a missing scale
    factor moves the analytic gradient far outside 4e-3 + 2e-2|n|;
  * float64 autograd of a two-pass softmax attention (torch on the CPU), an implementation
    independent of the oracle's loop nest, at several shapes, causal and not;
  * grouped == MHA over K/V repeated per query head with dK/dV summed over each group
    (src/backward_grouped.rs:214-245 compares grouped with the canonical oracle): a wrong
    query-head -> KV-head mapping fails it;
  * closed form seq_len = 1: P = 1, so dV = dO, dQ = dK = 0 exactly;
  * native KV-head cardinality of dK/dV (src/backward_grouped.rs:247-259);
  * threaded units reproduce the single-threaded result bit for bit.
"""
import numpy as np
import pytest

import oracle
from conftest import assert_close


def fixture(n, phase):
    """src/backward_grouped.rs:100-107."""
    x = np.arange(n, dtype=np.float32) * np.float32(0.31) + np.float32(phase)
    return (np.sin(x) * np.float32(0.65) + np.cos(x * np.float32(0.43)) * np.float32(0.23)
            ).astype(np.float32)


def _run(q, k, v, do, B, Hq, Hkv, S, D, causal, scale):
    o, lse = oracle.forward_grouped(q, k, v, B, Hq, Hkv, S, D, causal, scale)
    return oracle.backward_grouped(q, k, v, do, o, lse, B, Hq, Hkv, S, D, causal, scale)


@pytest.mark.parametrize("kv_heads,causal", [(2, True), (1, False), (4, True)])
def test_backward_matches_finite_differences(kv_heads, causal):
    B, Hq, S, D, scale = 1, 4, 3, 2, 0.67
    q = fixture(B * Hq * S * D, 0.1)
    k = fixture(B * kv_heads * S * D, 0.8)
    v = fixture(B * kv_heads * S * D, 1.4)
    do = fixture(B * Hq * S * D, 2.1)
    dq, dk, dv = _run(q, k, v, do, B, Hq, kv_heads, S, D, causal, scale)

    def objective(qq, kk, vv):
        o, _ = oracle.forward_grouped(qq, kk, vv, B, Hq, kv_heads, S, D, causal, scale)
        return float(np.sum(o * do, dtype=np.float32))

    eps = np.float32(1e-3)
    for name, analytic, which in (("dQ", dq, 0), ("dK", dk, 1), ("dV", dv, 2)):
        base = [q.copy(), k.copy(), v.copy()]
        num = np.zeros_like(analytic)
        for i in range(analytic.size):
            t = base[which]
            orig = t[i]
            t[i] = orig + eps
            plus = objective(*base)
            t[i] = orig - eps
            minus = objective(*base)
            t[i] = orig
            num[i] = (plus - minus) / (2.0 * eps)
        assert_close(name, analytic, num, 4e-3, 2e-2)


def _torch_grads(q, k, v, do, B, Hq, Hkv, S, D, causal, scale):
    torch = pytest.importorskip("torch")
    G = Hq // Hkv
    Q = torch.tensor(q.reshape(B, Hq, S, D), dtype=torch.float64, requires_grad=True)
    K = torch.tensor(k.reshape(B, Hkv, S, D), dtype=torch.float64, requires_grad=True)
    V = torch.tensor(v.reshape(B, Hkv, S, D), dtype=torch.float64, requires_grad=True)
    Ke = K.repeat_interleave(G, dim=1)
    Ve = V.repeat_interleave(G, dim=1)
    s = torch.einsum("bhqd,bhkd->bhqk", Q, Ke) * scale
    if causal:
        s = s.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool), 1), float("-inf"))
    o = torch.softmax(s, -1) @ Ve
    o.backward(torch.tensor(do.reshape(B, Hq, S, D), dtype=torch.float64))
    return [t.grad.numpy().ravel() for t in (Q, K, V)]


@pytest.mark.parametrize("B,Hq,Hkv,S,D,causal,scale", [
    (1, 1, 1, 1, 2, False, None),
    (1, 4, 4, 3, 8, True, None),
    (2, 8, 2, 5, 16, False, 0.23),
    (1, 8, 1, 9, 32, True, 0.17),
    (2, 12, 3, 7, 6, True, None),
    (1, 4, 2, 40, 64, True, None),
    (1, 2, 1, 33, 128, False, None),
])
def test_backward_matches_float64_autograd(B, Hq, Hkv, S, D, causal, scale):
    rng = np.random.default_rng(S * 131 + D)
    q = rng.standard_normal(B * Hq * S * D).astype(np.float32)
    k = rng.standard_normal(B * Hkv * S * D).astype(np.float32)
    v = rng.standard_normal(B * Hkv * S * D).astype(np.float32)
    do = rng.standard_normal(B * Hq * S * D).astype(np.float32)
    s = oracle.resolved_scale(D, scale)
    got = _run(q, k, v, do, B, Hq, Hkv, S, D, causal, s)
    want = _torch_grads(q, k, v, do, B, Hq, Hkv, S, D, causal, s)
    for name, a, e in zip(("dQ", "dK", "dV"), got, want):
        assert_close(name, a, e, 2e-5, 1e-4)


def test_grouped_equals_mha_over_repeated_kv():
    B, Hq, Hkv, S, D, causal = 2, 6, 2, 11, 8, True
    G = Hq // Hkv
    rng = np.random.default_rng(7)
    q = rng.standard_normal(B * Hq * S * D).astype(np.float32)
    k = rng.standard_normal(B * Hkv * S * D).astype(np.float32)
    v = rng.standard_normal(B * Hkv * S * D).astype(np.float32)
    do = rng.standard_normal(B * Hq * S * D).astype(np.float32)
    dq, dk, dv = _run(q, k, v, do, B, Hq, Hkv, S, D, causal, None)
    ke = np.repeat(k.reshape(B, Hkv, S, D), G, axis=1).ravel()
    ve = np.repeat(v.reshape(B, Hkv, S, D), G, axis=1).ravel()
    dq2, dk2, dv2 = _run(q, ke, ve, do, B, Hq, Hq, S, D, causal, None)
    np.testing.assert_array_equal(dq, dq2)
    assert_close("dK", dk, dk2.reshape(B, Hkv, G, S, D).sum(2, dtype=np.float32), 1e-6, 1e-5)
    assert_close("dV", dv, dv2.reshape(B, Hkv, G, S, D).sum(2, dtype=np.float32), 1e-6, 1e-5)


def test_single_key_closed_form():
    B, Hq, Hkv, S, D = 2, 4, 2, 1, 16
    rng = np.random.default_rng(3)
    q = rng.standard_normal(B * Hq * D).astype(np.float32)
    k = rng.standard_normal(B * Hkv * D).astype(np.float32)
    v = rng.standard_normal(B * Hkv * D).astype(np.float32)
    do = rng.standard_normal(B * Hq * D).astype(np.float32)
    dq, dk, dv = _run(q, k, v, do, B, Hq, Hkv, S, D, True, None)
    assert not dq.any() and not dk.any()
    # each KV head receives the sum over its group of dO, accumulated in query-head order
    want = np.zeros(B * Hkv * D, np.float32).reshape(B, Hkv, D)
    d3 = do.reshape(B, Hq, D)
    for b in range(B):
        for h in range(Hq):
            want[b, h // 2] += d3[b, h]
    np.testing.assert_array_equal(dv, want.ravel())


def test_native_kv_gradient_cardinality_and_threads():
    B, Hq, Hkv, S, D = 2, 8, 1, 4, 2
    q = fixture(B * Hq * S * D, 0.2)
    k = fixture(B * Hkv * S * D, 0.8)
    v = fixture(B * Hkv * S * D, 1.3)
    do = fixture(B * Hq * S * D, 1.9)
    o, lse = oracle.forward_grouped(q, k, v, B, Hq, Hkv, S, D, False)
    dq, dk, dv = oracle.backward_grouped(q, k, v, do, o, lse, B, Hq, Hkv, S, D, False)
    assert dq.size == q.size and dk.size == k.size and dv.size == v.size
    B, Hq, Hkv, S, D = 3, 8, 2, 17, 8
    rng = np.random.default_rng(1)
    xs = [rng.standard_normal(n).astype(np.float32)
          for n in (B * Hq * S * D, B * Hkv * S * D, B * Hkv * S * D, B * Hq * S * D)]
    o, lse = oracle.forward_grouped(xs[0], xs[1], xs[2], B, Hq, Hkv, S, D, True)
    one = oracle.backward_grouped(*xs, o, lse, B, Hq, Hkv, S, D, True, threads=1)
    many = oracle.backward_grouped(*xs, o, lse, B, Hq, Hkv, S, D, True, threads=4)
    for a, b in zip(one, many):
        np.testing.assert_array_equal(a, b)


def test_backward_rejects_bad_shapes():
    z = np.zeros(8, np.float32)
    with pytest.raises(oracle.OracleError) as e:
        oracle.backward_grouped(z, z, z, z, z, z, 1, 3, 2, 1, 2, False)
    assert e.value.code == 3
    with pytest.raises(oracle.OracleError) as e:
        oracle.backward_grouped(z, z, z, z, z, z, 1, 0, 1, 1, 2, False)
    assert e.value.code == 1
