"""GPU parity of the paged KV cache, split-K paged decode and paged chunked prefill.

Paged gather indexing is checked bit-exactly: the same data under a shuffled block table must
give bitwise identical output to the identity table. Numerics: f32 2e-5 + 1e-4|e|; bf16 2e-2.
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


def _fixture(n, phase):
    """Closed-form generator of tests/m16_paged_decode.rs:49-56."""
    x = np.arange(n, dtype=np.float32) * np.float32(0.021) + np.float32(phase)
    return (np.sin(x) * np.float32(1.1875) + np.cos(x * np.float32(0.43)) * np.float32(0.34375)).astype(np.float32)


def test_m16_paged_decode_matches_contiguous_oracle_across_page_boundaries(hip):
    """tests/m16_paged_decode.rs:171: Hq4 Hkv2 kv_len 7, page 3, 4 physical pages, D64, f32,
    unused rows filled with sentinels 17.0 / -19.0."""
    hq, hkv, kv_len, ps, pages, D, theta = 4, 2, 7, 3, 4, 64, 10000.0
    qpos = kv_len - 1
    q = _fixture(hq * D, 0.2)
    raw_k = _fixture(kv_len * hkv * D, 0.8)
    v = _fixture(kv_len * hkv * D, 1.4)
    eo, el = oracle.forward_projection_asymmetric(q, raw_k, v, 1, hq, hkv, 1, kv_len, D, qpos,
                                                  True, theta, qpos, 0, True)
    rot_k = oracle.rope_rotate_rows(raw_k, kv_len, hkv, D, theta)
    rows, width = ps * pages, hkv * D
    pk = np.full(rows * width, 17.0, np.float32)
    pv = np.full(rows * width, -19.0, np.float32)
    pk[:rot_k.size] = rot_k
    pv[:v.size] = v
    table = fa.PagedKvTable(fa.PagedKvConfig(ps, pages))
    table.append(kv_len)
    assert table.telemetry().mapped_pages == 3
    row = table.block_row()
    plan = fa.PagedDecodePlan(hip, row[None, :], np.array([kv_len]), ps, pages, hq, hkv, D,
                              fa.FlatAttentionConfig(True), theta, fa.DTYPE_F32,
                              q_positions=np.array([qpos]))
    qb, kb, vb = (fa.DeviceBuffer.from_array(hip, x) for x in (q, pk, pv))
    out = fa.DeviceBuffer(hip, plan.layout().combined_bytes)
    plan.launch(qb, kb, vb, out)
    res = fa.download_attention(out, plan.layout(), fa.DTYPE_F32)
    assert_close("paged O", res.output, eo, F32_ATOL, F32_RTOL)
    assert_close("paged LSE", res.lse, el, F32_ATOL, F32_RTOL)
    t = hip.last_telemetry()
    assert t.kernel_id == "DecodePagedSplitK" and t.dispatch_count == 2


def _make_pool(rng, ctx_lens, ps, hkv, D, rnd, shuffle=True, seed=7):
    pages_per = [(c + ps - 1) // ps for c in ctx_lens]
    total = sum(pages_per)
    ids = rng.permutation(total) if shuffle else np.arange(total)
    max_pages = max(pages_per)
    bt = np.zeros((len(ctx_lens), max_pages), np.int32)
    cur = 0
    for s, n in enumerate(pages_per):
        bt[s, :n] = ids[cur:cur + n]
        cur += n
    width = hkv * D
    kp = rnd(normal(total * ps * width, seed))
    vp = rnd(normal(total * ps * width, seed + 1))
    return bt, kp, vp, total


def _decode(hip, bt, ctx_lens, kp, vp, total, ps, hq, hkv, D, q, dtype, theta=1e4, split=None,
            causal=True):
    plan = fa.PagedDecodePlan(hip, bt, np.asarray(ctx_lens), ps, total, hq, hkv, D,
                              fa.FlatAttentionConfig(causal), theta, dtype)
    if split is not None:
        plan.set_split(split)
    qb, kb, vb = (fa.DeviceBuffer.from_array(hip, fa.host_storage(x, dtype)) for x in (q, kp, vp))
    out = fa.DeviceBuffer(hip, plan.layout().combined_bytes)
    plan.launch(qb, kb, vb, out)
    res = fa.download_attention(out, plan.layout(), dtype)
    return fa.storage_to_f32(res.output, dtype), res.lse, plan


@pytest.mark.parametrize("hq,hkv", [(32, 8), (8, 8), (32, 1), (12, 4)])
def test_batched_bf16_decode_matches_oracle(hip, hq, hkv):
    rng = np.random.default_rng(hq * 10 + hkv)
    ps, D = 16, 128
    ctx_lens = [1, 15, 16, 17, 100, 513, 1000, 2049]
    bt, kp, vp, total = _make_pool(rng, ctx_lens, ps, hkv, D, bf16_round)
    q = bf16_round(normal(len(ctx_lens) * hq * D, 3))
    o, l, _ = _decode(hip, bt, ctx_lens, kp, vp, total, ps, hq, hkv, D, q, fa.DTYPE_BF16)
    eo, el = oracle.paged_decode(q, kp, vp, total, ps, bt, ctx_lens, hq, hkv, D, True, 1e4)
    assert_close("O", o, eo, H16_ATOL, 0.0)
    assert_close("LSE", l, el, H16_ATOL, 0.0)


@pytest.mark.parametrize("dtype", [fa.DTYPE_BF16, fa.DTYPE_F16])
@pytest.mark.parametrize("ps,D,hq,hkv", [(16, 64, 8, 2), (32, 128, 16, 4), (48, 128, 8, 8),
                                         (5, 128, 8, 2), (24, 64, 4, 1), (16, 128, 32, 16)])
def test_16bit_decode_modes_match_oracle(hip, dtype, ps, D, hq, hkv):
    """16-bit KV in every decode layout: grouped MFMA (page size a multiple of 16, up to 8 KV
    heads), one-wave MFMA (more KV heads), VALU split-K (other page sizes); contexts ending
    inside pages and key steps."""
    rnd = bf16_round if dtype == fa.DTYPE_BF16 else f16_round
    rng = np.random.default_rng(ps * 3 + D + hkv)
    ctx_lens = [1, 17, 64, 95, 700]
    bt, kp, vp, total = _make_pool(rng, ctx_lens, ps, hkv, D, rnd, seed=ps + D)
    q = rnd(normal(len(ctx_lens) * hq * D, 5 + ps))
    o, l, _ = _decode(hip, bt, ctx_lens, kp, vp, total, ps, hq, hkv, D, q, dtype)
    t = hip.last_telemetry()
    assert t.kernel_id == ("DecodePagedMfma" if ps % 16 == 0 else "DecodePagedSplitK")
    eo, el = oracle.paged_decode(q, kp, vp, total, ps, bt, ctx_lens, hq, hkv, D, True, 1e4)
    assert_close("O", o, eo, H16_ATOL, 0.0)
    assert_close("LSE", l, el, H16_ATOL, 0.0)


@pytest.mark.parametrize("ps", [3, 16, 32])
@pytest.mark.parametrize("D", [64, 128])
def test_f32_decode_matches_oracle(hip, ps, D):
    rng = np.random.default_rng(ps + D)
    hq, hkv = 8, 2
    ctx_lens = [5, 48, 333, 900]
    bt, kp, vp, total = _make_pool(rng, ctx_lens, ps, hkv, D, lambda x: x)
    q = normal(len(ctx_lens) * hq * D, 4)
    o, l, _ = _decode(hip, bt, ctx_lens, kp, vp, total, ps, hq, hkv, D, q, fa.DTYPE_F32)
    eo, el = oracle.paged_decode(q, kp, vp, total, ps, bt, ctx_lens, hq, hkv, D, True, 1e4)
    assert_close("O", o, eo, F32_ATOL, F32_RTOL)
    assert_close("LSE", l, el, F32_ATOL, F32_RTOL)


def test_shuffled_block_table_is_bitwise_identical_to_identity(hip):
    """Same logical K/V rows placed under a shuffled vs identity page map."""
    rng = np.random.default_rng(3)
    ps, hq, hkv, D = 16, 32, 8, 128
    ctx_lens = [700, 1500, 33]
    bt_id, kp, vp, total = _make_pool(rng, ctx_lens, ps, hkv, D, bf16_round, shuffle=False)
    perm = rng.permutation(total)
    width = ps * hkv * D
    kp2 = np.empty_like(kp)
    vp2 = np.empty_like(vp)
    for logical_page in range(total):  # identity page p moves to physical perm[p]
        kp2[perm[logical_page] * width:(perm[logical_page] + 1) * width] = kp[logical_page * width:(logical_page + 1) * width]
        vp2[perm[logical_page] * width:(perm[logical_page] + 1) * width] = vp[logical_page * width:(logical_page + 1) * width]
    bt_sh = np.where(bt_id >= 0, perm[bt_id], 0).astype(np.int32)
    q = bf16_round(normal(len(ctx_lens) * hq * D, 9))
    o1, l1, _ = _decode(hip, bt_id, ctx_lens, kp, vp, total, ps, hq, hkv, D, q, fa.DTYPE_BF16)
    o2, l2, _ = _decode(hip, bt_sh, ctx_lens, kp2, vp2, total, ps, hq, hkv, D, q, fa.DTYPE_BF16)
    assert np.array_equal(o1.view(np.uint32), o2.view(np.uint32))
    assert np.array_equal(l1.view(np.uint32), l2.view(np.uint32))


def test_split_count_invariance(hip):
    rng = np.random.default_rng(5)
    ps, hq, hkv, D = 16, 32, 8, 128
    ctx_lens = [4000, 17, 1234]
    bt, kp, vp, total = _make_pool(rng, ctx_lens, ps, hkv, D, bf16_round)
    q = bf16_round(normal(len(ctx_lens) * hq * D, 2))
    ref = None
    for split in (16, 64, 256, 1008):
        o, l, plan = _decode(hip, bt, ctx_lens, kp, vp, total, ps, hq, hkv, D, q, fa.DTYPE_BF16,
                             split=split)
        assert plan.info()["split_tokens"] == split
        if ref is None:
            ref = (o, l)
        else:
            assert_close(f"O split {split}", o, ref[0], 1e-2, 0.0)
            assert_close(f"LSE split {split}", l, ref[1], 1e-4, 1e-5)


def test_cfg4_full_size_bf16_decode(hip):
    """64 sequences, ctx ~ U[512, 8192], page 16, Hq32 Hkv8 D128, bf16 KV,
    randomly permuted physical pages. Full oracle comparison."""
    rng = np.random.default_rng(2024)
    ps, hq, hkv, D = 16, 32, 8, 128
    ctx_lens = rng.integers(512, 8193, 64).tolist()
    bt, kp, vp, total = _make_pool(rng, ctx_lens, ps, hkv, D, bf16_round, seed=40)
    q = bf16_round(normal(64 * hq * D, 41))
    o, l, _ = _decode(hip, bt, ctx_lens, kp, vp, total, ps, hq, hkv, D, q, fa.DTYPE_BF16)
    eo, el = oracle.paged_decode(q, kp, vp, total, ps, bt, ctx_lens, hq, hkv, D, True, 1e4,
                                 threads=8)
    assert_close("O", o, eo, H16_ATOL, 0.0)
    assert_close("LSE", l, el, H16_ATOL, 0.0)


def test_decode_validation_errors(hip):
    bt = np.array([[0, 1]], np.int32)
    cfg = fa.FlatAttentionConfig(True)
    with pytest.raises(fa.FlatHipError) as e:
        fa.PagedDecodePlan(hip, bt, np.array([20]), 16, 2, 4, 2, 64, cfg, 1e4, fa.DTYPE_F32,
                           q_positions=np.array([10]))
    assert e.value.variant == "CausalVisibilityMismatch"
    with pytest.raises(fa.FlatHipError) as e:
        fa.PagedDecodePlan(hip, np.array([[0, 5]], np.int32), np.array([20]), 16, 2, 4, 2, 64,
                           cfg, 1e4, fa.DTYPE_F32)
    assert e.value.variant == "InvalidPage"
    with pytest.raises(fa.FlatHipError) as e:
        fa.PagedDecodePlan(hip, bt, np.array([0]), 16, 2, 4, 2, 64, cfg, 1e4, fa.DTYPE_F32)
    assert e.value.variant == "EmptyTable"
    with pytest.raises(fa.FlatHipError) as e:
        fa.PagedDecodePlan(hip, bt, np.array([20]), 16, 2, 4, 2, 64, cfg, float("nan"),
                           fa.DTYPE_F32)
    assert e.value.variant == "InvalidRotaryTheta"


# ------------------------------------------------------------------------------- cache


def test_paged_cache_append_crosses_pages_and_never_rewrites_prefix(hip):
    """tests/m16_paged_kv_cache.rs:159: appends split at page boundaries, prefix untouched."""
    ps, pages, hkv, D = 4, 5, 2, 16
    cache = fa.HipPagedKvCache(hip, fa.PagedKvConfig(ps, pages), hkv, D, fa.DTYPE_F32)
    width = hkv * D
    src_k1, src_v1 = normal(6 * width, 1), normal(6 * width, 2)
    src_k2, src_v2 = normal(5 * width, 3), normal(5 * width, 4)
    kb1, vb1 = fa.DeviceBuffer.from_array(hip, src_k1), fa.DeviceBuffer.from_array(hip, src_v1)
    assert cache.record_append(kb1, vb1, 6) == 6
    before = cache.k_buffer().download(np.float32, ps * pages * width).copy()
    kb2, vb2 = fa.DeviceBuffer.from_array(hip, src_k2), fa.DeviceBuffer.from_array(hip, src_v2)
    assert cache.record_append(kb2, vb2, 5) == 11
    kpool = cache.k_buffer().download(np.float32, ps * pages * width)
    vpool = cache.v_buffer().download(np.float32, ps * pages * width)
    table = cache.table()
    allk = np.concatenate([src_k1, src_k2]).reshape(11, width)
    allv = np.concatenate([src_v1, src_v2]).reshape(11, width)
    for tok in range(11):
        a = table.address(tok)
        r = a.physical_page * ps + a.offset_in_page
        assert np.array_equal(kpool[r * width:(r + 1) * width], allk[tok])
        assert np.array_equal(vpool[r * width:(r + 1) * width], allv[tok])
    for tok in range(6):  # prefix rows unchanged by the second append
        a = table.address(tok)
        r = a.physical_page * ps + a.offset_in_page
        assert np.array_equal(before[r * width:(r + 1) * width], kpool[r * width:(r + 1) * width])
    big_k = fa.DeviceBuffer.from_array(hip, normal(10 * width, 5))
    big_v = fa.DeviceBuffer.from_array(hip, normal(10 * width, 6))
    with pytest.raises(fa.FlatHipError) as e:
        cache.record_append(kb2, vb2, 10)  # source holds 5 rows: rejected before the table
    assert e.value.variant == "BufferTooSmall"
    with pytest.raises(fa.FlatHipError) as e:
        cache.record_append(big_k, big_v, 10)  # 21 > 20 tokens of capacity
    assert e.value.variant == "CapacityExceeded"
    assert len(cache.table()) == 11  # failed appends leave the table unchanged


def test_paged_cache_feeds_decode_with_rotate_on_append(hip):
    """Cache filled through rotate-on-append decodes like the raw-K asymmetric oracle."""
    ps, pages, hq, hkv, D, theta = 16, 8, 8, 2, 64, 1e4
    n = 75
    cache = fa.HipPagedKvCache(hip, fa.PagedKvConfig(ps, pages), hkv, D, fa.DTYPE_F32)
    raw_k, v = normal(n * hkv * D, 5), normal(n * hkv * D, 6)
    cache.record_append(fa.DeviceBuffer.from_array(hip, raw_k[:40 * hkv * D]),
                        fa.DeviceBuffer.from_array(hip, v[:40 * hkv * D]), 40,
                        rotate_k=fa.RotaryEmbeddingConfig(theta, 0))
    cache.record_append(fa.DeviceBuffer.from_array(hip, raw_k[40 * hkv * D:]),
                        fa.DeviceBuffer.from_array(hip, v[40 * hkv * D:]), n - 40,
                        rotate_k=fa.RotaryEmbeddingConfig(theta, 0))
    q = normal(hq * D, 7)
    pipe = fa.HipPagedDecodePipeline(hip, fa.DTYPE_F32)
    out = pipe.create_output_buffer(hq, D)
    lay = pipe.encode(fa.DeviceBuffer.from_array(hip, q), cache, out, hq,
                      fa.FlatAttentionConfig(True), theta, n - 1)
    res = fa.download_attention(out, lay, fa.DTYPE_F32)
    eo, el = oracle.forward_projection_asymmetric(q, raw_k, v, 1, hq, hkv, 1, n, D, n - 1, True,
                                                  theta, n - 1, 0, True)
    assert_close("O", res.output, eo, F32_ATOL, F32_RTOL)
    assert_close("LSE", res.lse, el, F32_ATOL, F32_RTOL)


def test_batched_append_scatter_is_bit_exact(hip):
    rng = np.random.default_rng(11)
    ps, hkv, D, n_seqs, app = 16, 8, 128, 4, 40
    starts = np.array([0, 5, 16, 31], np.int32)
    pages_per = [(s + app + ps - 1) // ps for s in starts]
    total = sum(pages_per) + 3
    ids = rng.permutation(total)
    bt = np.zeros((n_seqs, max(pages_per)), np.int32)
    cur = 0
    for s, n in enumerate(pages_per):
        bt[s, :n] = ids[cur:cur + n]
        cur += n
    width = hkv * D
    ks = bf16_round(normal(n_seqs * app * width, 1))
    vs = bf16_round(normal(n_seqs * app * width, 2))
    pool_el = total * ps * width
    kp = fa.DeviceBuffer(hip, pool_el * 2)
    vp = fa.DeviceBuffer(hip, pool_el * 2)
    kp.fill_u32(0)
    vp.fill_u32(0)
    fa.paged_append_batched(hip, bt, starts, app, ps, total, hkv, D,
                            fa.DeviceBuffer.from_array(hip, fa.host_storage(ks, fa.DTYPE_BF16)),
                            fa.DeviceBuffer.from_array(hip, fa.host_storage(vs, fa.DTYPE_BF16)),
                            kp, vp, None, fa.DTYPE_BF16)
    kpool = fa.bf16_bits_to_f32(kp.download(np.uint16, pool_el))
    vpool = fa.bf16_bits_to_f32(vp.download(np.uint16, pool_el))
    for s in range(n_seqs):
        for i in range(app):
            tok = int(starts[s]) + i
            r = bt[s, tok // ps] * ps + tok % ps
            src = (s * app + i) * width
            assert np.array_equal(kpool[r * width:(r + 1) * width], ks[src:src + width])
            assert np.array_equal(vpool[r * width:(r + 1) * width], vs[src:src + width])


@pytest.mark.parametrize("kernel", [-1, 0])
def test_cfg5_chunked_prefill_over_paged_cache(hip, kernel):
    """BASELINE configs[4] at its stated size: 8 sequences, each holding 2048 cached tokens + a
    new 512-token chunk in one shuffled page pool (page 16); the chunk attends causally at
    offset 2048 with Q RoPE at 2048 + i and pre-rotated K (rotate-on-append). The oracle checks
    the first and last head of the first and last sequence; V = 1 checks O = 1 on every row of
    every sequence and head (same Q/K, so LSE must repeat bit for bit)."""
    rng = np.random.default_rng(8)
    n_seqs, hq, hkv, D, ps, cached, ql, theta = 8, 32, 8, 128, 16, 2048, 512, 1e4
    kv_len = cached + ql
    pages_per = kv_len // ps
    total = n_seqs * pages_per
    bt = rng.permutation(total).astype(np.int32).reshape(n_seqs, pages_per)
    width = hkv * D
    raw_k = bf16_round(normal(n_seqs * kv_len * width, 1))
    v = bf16_round(normal(n_seqs * kv_len * width, 2))
    q = bf16_round(normal(n_seqs * ql * hq * D, 3))
    shape = fa.AsymmetricGroupedAttentionShape(n_seqs, hq, hkv, ql, kv_len, D, cached)
    plan = fa.PagedChunkedPrefillPlan(hip, bt, ps, total, shape, fa.FlatAttentionConfig(True),
                                      fa.AsymmetricRotaryEmbeddingConfig(theta, cached, 0),
                                      fa.DTYPE_BF16)
    qb = fa.DeviceBuffer.from_array(hip, fa.host_storage(q, fa.DTYPE_BF16))
    kb = fa.DeviceBuffer.from_array(hip, fa.host_storage(raw_k, fa.DTYPE_BF16))

    def run(v_host):
        kp = fa.DeviceBuffer(hip, total * ps * width * 2)
        vp = fa.DeviceBuffer(hip, total * ps * width * 2)
        fa.paged_append_batched(hip, bt, np.zeros(n_seqs, np.int32), kv_len, ps, total, hkv, D,
                                kb, fa.DeviceBuffer.from_array(hip, fa.host_storage(
                                    v_host, fa.DTYPE_BF16)),
                                kp, vp, fa.RotaryEmbeddingConfig(theta, 0), fa.DTYPE_BF16)
        out = fa.DeviceBuffer(hip, plan.layout().combined_bytes)
        plan.launch(qb, kp, vp, out)
        res = fa.download_attention(out, plan.layout(), fa.DTYPE_BF16)
        return fa.storage_to_f32(res.output, fa.DTYPE_BF16), res.lse

    hip.set_prefill_kernel(kernel)  # -1: the paged assembly kernel, 0: the HIP one
    try:
        o, lse = run(v)
        name = hip.last_telemetry().kernel_name
        assert ("prefill_a64" in name) == (kernel == -1), name
        o1, l1 = run(np.ones_like(v))
    finally:
        hip.set_prefill_kernel(-1)
    assert np.isfinite(o).all() and np.isfinite(lse).all()
    # oracle: RoPE materialised on Q (positions cached + i) and K (positions 0..kv_len-1) —
    # bit-exact to rotation inside the dot product (pinned in test_oracle.py) — then the
    # asymmetric oracle without RoPE on two head units per checked sequence.
    for s in (0, n_seqs - 1):
        sl_kv = slice(s * kv_len * width, (s + 1) * kv_len * width)
        qs = oracle.rope_rotate_rows(q[s * ql * hq * D:(s + 1) * ql * hq * D], ql, hq, D, theta,
                                     cached)
        ks = oracle.rope_rotate_rows(raw_k[sl_kv], kv_len, hkv, D, theta, 0)
        for unit in (0, hq - 1):
            eo, el = oracle.forward_projection_asymmetric(
                qs, ks, v[sl_kv], 1, hq, hkv, ql, kv_len, D, cached, True, None,
                units=(unit, unit + 1), threads=4)
            got = o[s * ql * hq * D:(s + 1) * ql * hq * D].reshape(ql, hq, D)[:, unit]
            exp = eo.reshape(ql, hq, D)[:, unit]
            assert_close(f"O seq {s} head {unit}", got, exp, H16_ATOL, 0.0)
            gl = lse[(s * hq + unit) * ql:(s * hq + unit + 1) * ql]
            assert_close(f"LSE seq {s} head {unit}", gl, el[unit * ql:(unit + 1) * ql], H16_ATOL, 0.0)
    assert np.max(np.abs(o1 - 1.0)) <= 2e-2
    assert np.array_equal(l1.view(np.uint32), lse.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("grouped", ["1", "0"])
def test_mixed_lengths_equal_work_partition_matches_oracle(hip, request, grouped):
    """Equal-work segment lists: 40 sequences from 1 to 3000 tokens, so some (sequence, head)
    units are finalised by one segment, others merge several partials, and one workgroup's range
    crosses sequence (and, with one-wave workgroups, head) boundaries. Both work layouts (the
    default head-grouped workgroups, and one-wave workgroups via fa_ctx_set_decode_policy(0)) are
    checked row by row against the oracle."""
    hip.set_decode_policy(-1 if grouped == "1" else 0)
    request.addfinalizer(lambda: hip.set_decode_policy(-1))
    rng = np.random.default_rng(21)
    ctx_lens = list(rng.integers(1, 3001, 40))
    ctx_lens[:4] = [1, 15, 16, 17]
    ps, hq, hkv, D = 16, 32, 8, 128
    bt, kp, vp, total = _make_pool(rng, ctx_lens, ps, hkv, D, bf16_round, seed=31)
    q = bf16_round(normal(len(ctx_lens) * hq * D, 33))
    o, lse, plan = _decode(hip, bt, ctx_lens, kp, vp, total, ps, hq, hkv, D, q, fa.DTYPE_BF16)
    info = plan.info()
    assert info["work_items"] > len(ctx_lens) * hkv  # some units are split
    eo, el = oracle.paged_decode(q, kp, vp, total, ps, bt, ctx_lens, hq, hkv, D, True, 1e4)
    assert_close("O", o, eo, H16_ATOL, 0.0)
    assert_close("LSE", lse, el, H16_ATOL, 0.0)


@pytest.mark.gpu
def test_kernel_timing_and_mfma_variant_telemetry(hip):
    """bf16 KV with page_size % 16 == 0 selects the MFMA split kernel; per-kernel timing counts
    one split and one combine dispatch per launch (the split kernel recording its events in its
    own dispatch, the results bitwise those without timing) and clears when re-enabled."""
    rng = np.random.default_rng(5)
    ctx_lens = [700, 1500, 33]
    ps, hq, hkv, D = 16, 8, 2, 128
    bt, kp, vp, total = _make_pool(rng, ctx_lens, ps, hkv, D, bf16_round)
    q = bf16_round(normal(len(ctx_lens) * hq * D, 3))
    o0, l0, _ = _decode(hip, bt, ctx_lens, kp, vp, total, ps, hq, hkv, D, q, fa.DTYPE_BF16)
    hip.set_kernel_timing(True)
    try:
        o1, l1, plan = _decode(hip, bt, ctx_lens, kp, vp, total, ps, hq, hkv, D, q,
                               fa.DTYPE_BF16)
        assert np.array_equal(np.asarray(o0).view(np.uint32), np.asarray(o1).view(np.uint32))
        assert np.array_equal(np.asarray(l0).view(np.uint32), np.asarray(l1).view(np.uint32))
        t = hip.last_telemetry()
        assert t.kernel_id == "DecodePagedMfma" and t.dispatch_count == 2
        ms, n = hip.kernel_timing("DecodePagedMfma")
        assert n == 1 and ms > 0.0
        assert hip.kernel_timing_range("DecodePagedMfma") == (ms, ms)  # one dispatch
        ms, n = hip.kernel_timing("DecodeCombine")
        assert n == 1 and ms > 0.0
        assert hip.kernel_timing("DecodePagedSplitK") == (0.0, 0)
        hip.set_kernel_timing(True)
        assert hip.kernel_timing("DecodePagedMfma") == (0.0, 0)
        assert hip.kernel_timing_range("DecodePagedMfma") == (0.0, 0.0)
    finally:
        hip.set_kernel_timing(False)


def _paged_prefill(hip, bt, ps, total, n_seqs, hq, hkv, D, cached, ql, theta, raw_k, v, q, dtype,
                   causal, pools=None):
    kv_len = cached + ql
    kp = fa.DeviceBuffer(hip, total * ps * hkv * D * 4)
    vp = fa.DeviceBuffer(hip, total * ps * hkv * D * 4)
    kp.fill_u32(0x7FC00000)  # pool rows no table names hold NaN: a wrong gather shows
    fa.paged_append_batched(hip, bt, np.zeros(n_seqs, np.int32), kv_len, ps, total, hkv, D,
                            fa.DeviceBuffer.from_array(hip, fa.host_storage(raw_k, dtype)),
                            fa.DeviceBuffer.from_array(hip, fa.host_storage(v, dtype)),
                            kp, vp, fa.RotaryEmbeddingConfig(theta, 0), dtype)
    shape = fa.AsymmetricGroupedAttentionShape(n_seqs, hq, hkv, ql, kv_len, D, cached)
    plan = fa.PagedChunkedPrefillPlan(hip, bt, ps, total, shape, fa.FlatAttentionConfig(causal),
                                      fa.AsymmetricRotaryEmbeddingConfig(theta, cached, 0), dtype)
    out = fa.DeviceBuffer(hip, plan.layout().combined_bytes)
    plan.launch(fa.DeviceBuffer.from_array(hip, fa.host_storage(q, dtype)), kp, vp, out)
    res = fa.download_attention(out, plan.layout(), dtype)
    if pools is not None:  # the pools as the device holds them (pre-rotated K), in f32
        n = total * ps * hkv * D
        sd = {fa.DTYPE_F32: np.float32, fa.DTYPE_BF16: np.uint16, fa.DTYPE_F16: np.uint16}[dtype]
        pools.extend(fa.storage_to_f32(b.download(sd, n), dtype) for b in (kp, vp))
    return fa.storage_to_f32(res.output, dtype), res.lse


@pytest.mark.parametrize("dtype", [fa.DTYPE_BF16, fa.DTYPE_F16, fa.DTYPE_F32])
@pytest.mark.parametrize("ps", [16, 5, 32])
@pytest.mark.parametrize("D,causal", [(128, True), (64, True), (128, False)])
def test_paged_prefill_modes_match_oracle_and_gather_bit_exactly(hip, dtype, ps, D, causal):
    """Chunked prefill over the paged cache in every addressing mode: 16-bit with page size a
    multiple of 16 (one page per 16-key group, 8-wave ping-pong kernel), 16-bit with any page
    size (4-wave kernel), and f32. A query
    chunk of 50 rows after 37 cached tokens, so key tiles and pages end mid-way. The same
    data under the identity block table and a shuffled one must give bitwise identical O/LSE."""
    rnd = {fa.DTYPE_BF16: bf16_round, fa.DTYPE_F16: f16_round, fa.DTYPE_F32: lambda x: x}[dtype]
    atol, rtol = (F32_ATOL, F32_RTOL) if dtype == fa.DTYPE_F32 else (H16_ATOL, 0.0)
    n_seqs, hq, hkv, cached, ql, theta = 2, 8, 2, 37, 50, 1e4
    kv_len = cached + ql
    pages_per = -(-kv_len // ps)
    total = n_seqs * pages_per + 3  # a few pool pages no table names
    rng = np.random.default_rng(ps * 7 + D)
    width = hkv * D
    raw_k = rnd(normal(n_seqs * kv_len * width, 31 + ps))
    v = rnd(normal(n_seqs * kv_len * width, 32 + ps))
    q = rnd(normal(n_seqs * ql * hq * D, 33 + ps))
    ident = np.arange(n_seqs * pages_per, dtype=np.int32).reshape(n_seqs, pages_per)
    shuf = rng.permutation(total)[:n_seqs * pages_per].astype(np.int32).reshape(n_seqs, pages_per)
    o1, l1 = _paged_prefill(hip, ident, ps, total, n_seqs, hq, hkv, D, cached, ql, theta, raw_k,
                            v, q, dtype, causal)
    t = hip.last_telemetry()
    if dtype != fa.DTYPE_F32 and ps == 16 and D == 128:  # the paged assembly kernel
        assert "prefill_a64" in t.kernel_name and t.workgroup_size == 256, t.kernel_name
    elif dtype != fa.DTYPE_F32:  # page % 16 == 0: 8-wave ping-pong kernel; else the 4-wave one
        assert t.workgroup_size == (512 if ps % 16 == 0 else 256)
    pools = []
    o2, l2 = _paged_prefill(hip, shuf, ps, total, n_seqs, hq, hkv, D, cached, ql, theta, raw_k,
                            v, q, dtype, causal, pools)
    assert np.array_equal(o1.view(np.uint32), o2.view(np.uint32))
    assert np.array_equal(l1.view(np.uint32), l2.view(np.uint32))
    # the paged oracle over the device's own shuffled pool (pre-rotated K as appended): checks
    # the gather and the Q rotation independently of the append's rounding of rotated K
    po, pl = oracle.paged_prefill(q, pools[0], pools[1], total, ps, shuf, hq, hkv, ql, kv_len, D,
                                  cached, causal, theta, cached, threads=2)
    assert_close("O vs paged oracle", o2, po, atol, rtol)
    assert_close("LSE vs paged oracle", l2, pl, atol, rtol)
    for s in range(n_seqs):
        sl_kv = slice(s * kv_len * width, (s + 1) * kv_len * width)
        qs = oracle.rope_rotate_rows(q[s * ql * hq * D:(s + 1) * ql * hq * D], ql, hq, D, theta,
                                     cached)
        ks = oracle.rope_rotate_rows(raw_k[sl_kv], kv_len, hkv, D, theta, 0)
        eo, el = oracle.forward_projection_asymmetric(qs, ks, v[sl_kv], 1, hq, hkv, ql, kv_len,
                                                      D, cached, causal, None)
        assert_close(f"O seq {s}", o1[s * ql * hq * D:(s + 1) * ql * hq * D], eo, atol, rtol)
        assert_close(f"LSE seq {s}", l1[s * hq * ql:(s + 1) * hq * ql], el, atol, rtol)


@pytest.mark.parametrize("pattern", ["rising", "falling", "alternating"])
@pytest.mark.parametrize("dtype", [fa.DTYPE_BF16, fa.DTYPE_F16])
@pytest.mark.parametrize("layout", ["1", "0"])
@pytest.mark.parametrize("split", [None, 256])
def test_adversarial_scores_16bit_decode(hip, request, pattern, dtype, layout, split):
    """Split-K decode with scores that rise over the whole context (every segment's maximum
    exceeds the previous ones, so the combine rescales every partial), fall (later segments'
    probabilities underflow), or alternate between +-24; in both 16-bit formats, both MFMA work
    layouts (head-grouped workgroups and one-wave workgroups, fa_ctx_set_decode_policy(0)) and with the
    automatic and an explicit split, so every kernel variant that carries the rotated query's
    residual operand is covered."""
    hip.set_decode_policy(-1 if layout == "1" else 0)
    request.addfinalizer(lambda: hip.set_decode_policy(-1))
    rnd = bf16_round if dtype == fa.DTYPE_BF16 else f16_round
    ps, hq, hkv, D = 16, 4, 1, 128
    ctx_lens = [2000, 700]
    rng = np.random.default_rng(11)
    bt, kp, vp, total = _make_pool(rng, ctx_lens, ps, hkv, D, rnd, seed=12)
    kp = kp.reshape(total * ps, hkv, D)
    kp[:] = 0.0
    for s, n in enumerate(ctx_lens):
        idx = np.arange(n, dtype=np.float32)
        sc = {"rising": 0.05 * idx, "falling": -0.05 * idx,
              "alternating": np.where(np.arange(n) % 3 == 0, 24.0, -24.0)}[pattern]
        rows = bt[s, np.arange(n) // ps] * ps + np.arange(n) % ps
        kp[rows, :, 0] = (sc * np.sqrt(D))[:, None]
    kp = rnd(kp.ravel())
    q = np.zeros((len(ctx_lens), hq, D), np.float32)
    q[:, :, 0] = 1.0
    q = q.ravel()
    o, l, plan = _decode(hip, bt, ctx_lens, kp, vp, total, ps, hq, hkv, D, q, dtype, split=split)
    t = hip.last_telemetry()
    assert t.kernel_id == "DecodePagedMfma"
    # head-grouped workgroups run with the automatic split only
    assert ("grouped" in t.kernel_name) == (layout == "1" and split is None), t.kernel_name
    eo, el = oracle.paged_decode(q, kp, vp, total, ps, bt, ctx_lens, hq, hkv, D, True, 1e4)
    assert np.isfinite(o).all() and np.isfinite(l).all()
    assert_close("O", o, eo, H16_ATOL, 0.0)
    # scores near 60: a once-rounded rotated query would move LSE by ~0.2; the decode keeps the
    # query's residual as a second MFMA operand, so LSE stays within the 16-bit bar
    assert_close("LSE", l, el, H16_ATOL, 0.0)
