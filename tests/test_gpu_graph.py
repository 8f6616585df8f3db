"""HIP graphs over the library's launches (fa_graph_*; no counterpart in the reference, whose
callers record passes into a command encoder and submit it).

A prepared paged decode, a prepared contiguous forward (K pre-rotation pass + prefill) and a
prepared recompute backward (delta, the assembly dK/dV kernel, dQ from the stored dS) are
captured once and replayed several times with new buffer contents between replays and eager
work and synchronisations in between; every replay must give the same bits as an eager launch
on the same inputs. Calls that would allocate, upload, fill or wait are refused while
capturing and leave the capture usable.
"""
import numpy as np
import pytest

from _inputs import bf16_round, normal

import flat_attention_amd as fa

pytestmark = pytest.mark.gpu


def _bits(buf, n):
    return buf.download(np.uint8, n)


def test_captured_paged_decode_replays_match_eager(hip):
    rng = np.random.default_rng(11)
    ctx_lens = np.array([700, 1500, 33, 1024], np.int32)
    ps, hq, hkv, D = 16, 8, 2, 128
    pages = (ctx_lens + ps - 1) // ps
    total = int(pages.sum())
    ids = rng.permutation(total)
    bt = np.zeros((len(ctx_lens), int(pages.max())), np.int32)
    cur = 0
    for s, n in enumerate(pages):
        bt[s, :n] = ids[cur:cur + n]
        cur += n
    width = hkv * D
    dt = fa.DTYPE_BF16
    kb = fa.DeviceBuffer.from_array(hip, fa.host_storage(normal(total * ps * width, 1), dt))
    vb = fa.DeviceBuffer.from_array(hip, fa.host_storage(normal(total * ps * width, 2), dt))
    plan = fa.PagedDecodePlan(hip, bt, ctx_lens, ps, total, hq, hkv, D,
                              fa.FlatAttentionConfig(True), 1e4, dt)
    nq = len(ctx_lens) * hq * D
    qb = fa.DeviceBuffer(hip, nq * 2)
    out_g = fa.DeviceBuffer(hip, plan.layout().combined_bytes)
    out_e = fa.DeviceBuffer(hip, plan.layout().combined_bytes)
    qb.upload(fa.host_storage(bf16_round(normal(nq, 3)), dt))
    plan.launch(qb, kb, vb, out_e)  # warms the RoPE table cache before capturing
    with hip.capture() as cap:
        plan.launch(qb, kb, vb, out_g)
    n = plan.layout().combined_bytes
    for rep in range(3):
        qb.upload(fa.host_storage(bf16_round(normal(nq, 10 + rep)), dt))
        cap.graph.launch()
        plan.launch(qb, kb, vb, out_e)
        hip.synchronize()
        assert np.array_equal(_bits(out_g, n), _bits(out_e, n)), rep
        res = fa.download_attention(out_g, plan.layout(), dt)
        assert np.all(np.isfinite(res.lse))


def test_captured_prepared_forward_replays_match_eager(hip):
    B, hq, hkv, S, D = 1, 8, 2, 300, 128
    shape = fa.GroupedAttentionShape(B, hq, hkv, S, D)
    cfg = fa.FlatAttentionConfig(True)
    rot = fa.RotaryEmbeddingConfig(1e4, 5)
    ex = fa.HipRotaryGroupedAttention(hip, fa.DTYPE_BF16)
    bq = ex.upload(normal(shape.q_tensor_len(), 1))
    bk = ex.upload(normal(shape.kv_tensor_len(), 2))
    bv = ex.upload(normal(shape.kv_tensor_len(), 3))
    n = ex.layout(shape).combined_bytes
    out_g, out_e = fa.DeviceBuffer(hip, n), fa.DeviceBuffer(hip, n)
    prep = ex.prepare(bq, bk, bv, out_g, shape, cfg, rot)
    with hip.capture() as cap:
        ex.encode_prepared(prep)
    assert hip.last_telemetry().dispatch_count == 2  # rotate_rows + prefill, recorded
    for rep in range(3):
        bk.upload(fa.host_storage(normal(shape.kv_tensor_len(), 20 + rep), fa.DTYPE_BF16))
        cap.graph.launch()
        ex.forward_resident(bq, bk, bv, shape, cfg, rot, out_e)
        hip.synchronize()
        assert np.array_equal(_bits(out_g, n), _bits(out_e, n)), rep


def test_captured_backward_replays_match_eager(hip):
    """The default bf16 backward (bwd_delta + fa_bwd_dkdv_a64_bf16 + bwd_dq_ds): its workspaces
    are grown by an eager call first, so the captured call records only the three launches."""
    import oracle
    B, hq, hkv, S, D = 1, 8, 2, 256, 128
    shape = fa.GroupedAttentionShape(B, hq, hkv, S, D)
    cfg = fa.FlatAttentionConfig(True)
    dt = fa.DTYPE_BF16
    q, k, v, do = (bf16_round(normal(n, 40 + i)) for i, n in enumerate(
        (B * hq * S * D, B * hkv * S * D, B * hkv * S * D, B * hq * S * D)))
    o, lse = oracle.forward_grouped(q, k, v, B, hq, hkv, S, D, True)
    pipe = fa.HipGroupedBackwardRecomputePipeline(hip, dt)
    lay = pipe.layout(shape)
    fwd = fa.DeviceBuffer.from_array(hip, fa.pack_grouped_backward_recompute_inputs(
        q, k, v, do, fa.FlatAttentionOutput(bf16_round(o), lse), shape, dt, lay))
    g_graph, g_eager = pipe.create_gradient_buffer(shape), pipe.create_gradient_buffer(shape)
    prep = pipe.prepare(fwd, g_graph, shape, cfg)
    pipe.encode(fwd, g_eager, shape, cfg)  # grows the delta and dS workspaces
    with hip.capture() as cap:
        pipe.encode_prepared(prep)
    assert "bwd_dkdv_a64" in hip.last_telemetry().kernel_name
    n = lay.gradient_bytes
    for rep in range(3):
        new_do = fa.host_storage(bf16_round(normal(B * hq * S * D, 50 + rep)), dt)
        fwd.upload(new_do, lay.d_out_offset)
        cap.graph.launch()
        pipe.encode(fwd, g_eager, shape, cfg)
        hip.synchronize()
        assert np.array_equal(_bits(g_graph, n), _bits(g_eager, n)), rep
        res = pipe.download_gradients(g_graph, shape)
        assert all(np.isfinite(x).all() for x in (res.dq, res.dk, res.dv))


def test_capture_refuses_allocation_upload_fill_and_wait(hip):
    fresh = fa.HipContext(0)
    try:
        buf = fa.DeviceBuffer(fresh, 1024)
        ex = fa.HipRotaryGroupedAttention(fresh, fa.DTYPE_BF16)
        shape = fa.GroupedAttentionShape(1, 4, 2, 64, 64)
        q = ex.upload(normal(shape.q_tensor_len(), 1))
        kv = ex.upload(normal(shape.kv_tensor_len(), 2))
        out = fa.DeviceBuffer(fresh, ex.layout(shape).combined_bytes)
        bt = np.zeros((1, 1), np.int32)
        lens = np.array([16], np.int32)
        dq = fa.DeviceBuffer(fresh, 4 * 64 * 2)
        dkv = fa.DeviceBuffer(fresh, 16 * 2 * 64 * 2)
        dout = fa.DeviceBuffer(fresh, fa.packed_layout(4 * 64, 4, fa.DTYPE_BF16).combined_bytes)
        with fresh.capture() as cap:
            for call in (lambda: buf.fill_u32(0),
                         lambda: hip_sync(fresh),
                         # the allocation-free decode copies its metadata from a host area
                         lambda: fa.paged_decode_noalloc(fresh, bt, lens, 16, 1, 4, 2, 64,
                                                         fa.FlatAttentionConfig(True), 1e4,
                                                         fa.DTYPE_BF16, dq, dkv, dkv, dout),
                         # cold context: the RoPE table and K workspace would be allocated
                         lambda: ex.forward_resident(q, kv, kv, shape, fa.FlatAttentionConfig(True),
                                                     fa.RotaryEmbeddingConfig(1e4, 0), out)):
                with pytest.raises(fa.FlatHipError) as e:
                    call()
                assert e.value.variant == "GraphCapture", e.value
            with pytest.raises(fa.FlatHipError) as e:
                fresh.capture_begin()
            assert e.value.variant == "GraphCapture"
        cap.graph.launch()  # an empty graph
        fresh.synchronize()
    finally:
        fresh.close()


def hip_sync(ctx):
    ctx.synchronize()
