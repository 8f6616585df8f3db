"""GPU parity of the allocation-free paged decode (fa_paged_decode_noalloc) against the
prepared decode (fa_paged_decode_prepare + fa_paged_decode_launch): same kernels, so the bar is
bitwise identity of O and LSE. Two calls in a row share the device's static scratch, the second
with a smaller input, so stale scratch contents from the first must not leak into the second.
"""
import numpy as np
import pytest

from _inputs import bf16_round, f16_round, normal

import flat_attention_amd as fa

pytestmark = pytest.mark.gpu

ROUND = {fa.DTYPE_BF16: bf16_round, fa.DTYPE_F16: f16_round, fa.DTYPE_F32: lambda x: x}


def _pool(rng, ctx_lens, ps, hkv, D, rnd, seed):
    pages_per = [(c + ps - 1) // ps for c in ctx_lens]
    total = sum(pages_per)
    ids = rng.permutation(total)
    bt = np.zeros((len(ctx_lens), max(pages_per)), np.int32)
    cur = 0
    for s, n in enumerate(pages_per):
        bt[s, :n] = ids[cur:cur + n]
        cur += n
    kp = rnd(normal(total * ps * hkv * D, seed))
    vp = rnd(normal(total * ps * hkv * D, seed + 1))
    return bt, kp, vp, total


def _both(hip, ctx_lens, ps, hq, hkv, D, dtype, seed, q_positions=None):
    """Runs the prepared decode and the allocation-free one on the same inputs; returns the two
    packed outputs as raw bytes and the allocation-free call's telemetry."""
    rng = np.random.default_rng(seed)
    rnd = ROUND[dtype]
    bt, kp, vp, total = _pool(rng, ctx_lens, ps, hkv, D, rnd, seed)
    lens = np.asarray(ctx_lens, np.int32)
    q = rnd(normal(len(ctx_lens) * hq * D, seed + 2))
    cfg = fa.FlatAttentionConfig(True)
    qb, kb, vb = (fa.DeviceBuffer.from_array(hip, fa.host_storage(x, dtype)) for x in (q, kp, vp))
    plan = fa.PagedDecodePlan(hip, bt, lens, ps, total, hq, hkv, D, cfg, 1e4, dtype,
                              q_positions=q_positions)
    lay = plan.layout()
    ref = fa.DeviceBuffer(hip, lay.combined_bytes)
    ref.fill_u32(0x7FC00001)
    plan.launch(qb, kb, vb, ref)
    got = fa.DeviceBuffer(hip, lay.combined_bytes)
    got.fill_u32(0x7FC00002)
    lay2 = fa.paged_decode_noalloc(hip, bt, lens, ps, total, hq, hkv, D, cfg, 1e4, dtype, qb, kb,
                                   vb, got, q_positions=q_positions)
    tel = hip.last_telemetry()
    assert lay2.combined_bytes == lay.combined_bytes
    a = ref.download(np.uint8, lay.combined_bytes)
    b = got.download(np.uint8, lay.combined_bytes)
    return a, b, tel, plan.info()


def _assert_identical(a, b):
    diff = np.flatnonzero(a != b)
    assert diff.size == 0, f"{diff.size} bytes differ, first at {diff[:8]}"


@pytest.mark.parametrize("dtype", [fa.DTYPE_BF16, fa.DTYPE_F16, fa.DTYPE_F32])
def test_noalloc_decode_matches_prepared_decode_on_two_calls(hip, dtype):
    """First a larger batch (several split segments per sequence), then a smaller one."""
    ps = 16 if dtype != fa.DTYPE_F32 else 5
    a, b, tel, _ = _both(hip, [3000, 17, 1, 4100, 700, 2049, 64, 5000], ps, 32, 8, 128, dtype, 11)
    _assert_identical(a, b)
    assert tel.temporary_allocation_count == 0
    a, b, tel, _ = _both(hip, [33, 900, 16], ps, 8, 2, 64, dtype, 12,
                         q_positions=np.array([40, 900, 2000], np.int32))
    _assert_identical(a, b)
    assert tel.temporary_allocation_count == 0


def test_noalloc_decode_cfg4_then_smaller(hip):
    """BASELINE configs[3] at full size (64 sequences, ctx ~ U[512, 8192], page 16, Hq32 Hkv8
    D128, bf16, shuffled pages) through the scratch, then a 5-sequence batch."""
    rng = np.random.default_rng(2024)
    ctx_lens = rng.integers(512, 8193, 64).tolist()
    a, b, tel, info = _both(hip, ctx_lens, 16, 32, 8, 128, fa.DTYPE_BF16, 40)
    _assert_identical(a, b)
    assert tel.kernel_id == "DecodePagedMfma"
    assert tel.temporary_allocation_count == 0
    print(f"cfg4 partials {info['workspace_bytes']} bytes", flush=True)
    a, b, tel, _ = _both(hip, [513, 1, 8000, 47, 2048], 16, 32, 8, 128, fa.DTYPE_BF16, 41)
    _assert_identical(a, b)


def test_noalloc_decode_rejects_oversized_metadata_before_device_work(hip):
    """Block tables beyond the scratch's 4 MiB metadata part fail with ScratchExceeded, and a
    valid call afterwards still matches the prepared decode."""
    hq, hkv, D, ps = 8, 2, 64, 16
    bt = np.zeros((1, 1_100_000), np.int32)
    lens = np.array([16], np.int32)
    q = fa.DeviceBuffer(hip, hq * D * 2)
    kv = fa.DeviceBuffer(hip, ps * hkv * D * 2)
    out = fa.DeviceBuffer(hip, fa.packed_layout(hq * D, hq, fa.DTYPE_BF16).combined_bytes)
    with pytest.raises(fa.FlatHipError) as e:
        fa.paged_decode_noalloc(hip, bt, lens, ps, 1, hq, hkv, D, fa.FlatAttentionConfig(True),
                                1e4, fa.DTYPE_BF16, q, kv, kv, out)
    assert e.value.variant == "ScratchExceeded"
    a, b, _, _ = _both(hip, [100, 250], ps, hq, hkv, D, fa.DTYPE_BF16, 13)
    _assert_identical(a, b)


def test_noalloc_decode_two_contexts_interleaved(hip):
    """Two contexts (two streams) on one GPU share the device's scratch. Calls issued back to
    back from both, with no host synchronisation between them, are ordered on the GPU by the
    scratch's last-user event: each output is bitwise equal to the prepared decode's."""
    other = fa.HipContext(0)
    try:
        cases = []
        for i, (lens, hq, hkv, D) in enumerate(
                [([3000, 17, 4100, 700, 5000, 2049], 32, 8, 128), ([33, 900, 16], 8, 2, 64),
                 ([8000, 512, 1], 32, 8, 128), ([65, 4000], 16, 4, 128)]):
            rng = np.random.default_rng(70 + i)
            bt, kp, vp, total = _pool(rng, lens, 16, hkv, D, bf16_round, 70 + i)
            cl = np.asarray(lens, np.int32)
            q = bf16_round(normal(len(lens) * hq * D, 80 + i))
            cfg = fa.FlatAttentionConfig(True)
            ctx = hip if i % 2 == 0 else other
            qb, kb, vb = (fa.DeviceBuffer.from_array(ctx, fa.host_storage(x, fa.DTYPE_BF16))
                          for x in (q, kp, vp))
            plan = fa.PagedDecodePlan(hip, bt, cl, 16, total, hq, hkv, D, cfg, 1e4, fa.DTYPE_BF16)
            lay = plan.layout()
            ref = fa.DeviceBuffer(hip, lay.combined_bytes)
            q_ref, k_ref, v_ref = (fa.DeviceBuffer.from_array(hip, fa.host_storage(x, fa.DTYPE_BF16))
                                   for x in (q, kp, vp))
            plan.launch(q_ref, k_ref, v_ref, ref)
            got = fa.DeviceBuffer(ctx, lay.combined_bytes)
            got.fill_u32(0x7FC00003)
            cases.append((ctx, bt, cl, total, hq, hkv, D, cfg, qb, kb, vb, got, ref, lay))
        hip.synchronize()
        other.synchronize()
        for _ in range(3):  # interleaved, no host wait between the calls
            for (ctx, bt, cl, total, hq, hkv, D, cfg, qb, kb, vb, got, ref, lay) in cases:
                fa.paged_decode_noalloc(ctx, bt, cl, 16, total, hq, hkv, D, cfg, 1e4,
                                        fa.DTYPE_BF16, qb, kb, vb, got)
        for n, (ctx, *_, got, ref, lay) in enumerate(cases):
            a = ref.download(np.uint8, lay.combined_bytes)
            b = got.download(np.uint8, lay.combined_bytes)
            print(f"two-context case {n}", flush=True)
            _assert_identical(a, b)
    finally:
        other.synchronize()
        other.close()
