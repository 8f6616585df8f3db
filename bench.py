#!/usr/bin/env python3
"""Benchmark of the FLAT-ATTENTION hot path on one MI355X.

One step = one causal GQA prefill with fused RoPE on BASELINE configs[2]
(B2 Hq32 Hkv8 N4096 D128, bf16 storage, f32 accumulation) followed by one split-K paged decode
on configs[3] (64 sequences, ctx ~ U[512, 8192], page 16, Hq32 Hkv8 D128, bf16 KV, shuffled
page pool). Inputs are synthetic and resident in HBM before timing. Each op is bracketed by
HIP events recorded on the library's own stream.

value = prefill TFLOP/s (algorithmic FLOP over visible (q, k) pairs: 4*B*Hq*D*N(N+1)/2);
decode GB/s (algorithmic bytes: K+V of every live token once, plus Q, O, LSE, block tables)
is reported beside it with its own roofline. `value` and each op's rate use the op's whole
duration (the prefill op includes the K pre-rotation pass); each `roofline.achieved` divides the
same algorithmic work by the average duration of the op's dominant kernel alone, timed by the
library's per-dispatch events (fa_ctx_set_kernel_timing) in the same timed steps, so both
figures describe the same clocks.
`roofline.traffic` is the HBM bytes
per launch of that kernel from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary
(profiles/hbm_traffic_prefill_decode.json), scaled by a 1 GiB device-copy calibration.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "flat-attention_amd"))

import flat_attention_amd as fa  # noqa: E402

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E


class HipEvents:
    """hipEvent timing on an arbitrary stream (libamdhip64 via ctypes)."""

    def __init__(self):
        self.h = ctypes.CDLL("libamdhip64.so")
        self.h.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.h.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.h.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.h.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                               ctypes.c_void_p]
        self.h.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.h.hipMemcpyAsync.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                          ctypes.c_int, ctypes.c_void_p]

    def copy_d2d(self, dst, src, nbytes, stream):
        assert self.h.hipMemcpyAsync(dst, src, nbytes, 3, ctypes.c_void_p(stream)) == 0

    def create(self):
        e = ctypes.c_void_p()
        assert self.h.hipEventCreate(ctypes.byref(e)) == 0
        return e

    def record(self, e, stream):
        assert self.h.hipEventRecord(e, ctypes.c_void_p(stream)) == 0

    def elapsed_ms(self, a, b):
        assert self.h.hipEventSynchronize(b) == 0
        ms = ctypes.c_float()
        assert self.h.hipEventElapsedTime(ctypes.byref(ms), a, b) == 0
        return ms.value


def bf16_normal(rng, n):
    return fa.f32_to_bf16_bits(rng.standard_normal(n, dtype=np.float32))


def build_prefill(ctx, rng, data="normal"):
    B, hq, hkv, S, D = 2, 32, 8, 4096, 128
    shape = fa.GroupedAttentionShape(B, hq, hkv, S, D)
    ex = fa.HipRotaryGroupedAttention(ctx, fa.DTYPE_BF16)
    if data == "constant":
        # power-limit diagnostic: the same instruction stream and memory traffic on data whose
        # MFMA operands never toggle
        fill = lambda n: fa.f32_to_bf16_bits(np.full(n, 0.5, np.float32))  # noqa: E731
    else:
        fill = lambda n: bf16_normal(rng, n)  # noqa: E731
    q = fa.DeviceBuffer.from_array(ctx, fill(shape.q_tensor_len()))
    k = fa.DeviceBuffer.from_array(ctx, fill(shape.kv_tensor_len()))
    v = fa.DeviceBuffer.from_array(ctx, fill(shape.kv_tensor_len()))
    out = fa.DeviceBuffer(ctx, ex.layout(shape).combined_bytes)
    cfg = fa.FlatAttentionConfig(causal=True)
    rot = fa.RotaryEmbeddingConfig(10000.0, 0)
    flop = 4.0 * B * hq * D * S * (S + 1) / 2
    # the prepared forward (PreparedGroupedForward::prepare / encode_prepared): a step only
    # enqueues the K rotation pass and the prefill kernel
    prep = ex.prepare(q, k, v, out, shape, cfg, rot)
    run = lambda: ex.encode_prepared(prep)  # noqa: E731
    run._keep = prep
    return run, flop, {"workload": "prefill: causal GQA+RoPE B2 Hq32 Hkv8 N4096 D128 bf16",
                       "flop_per_step": flop, "entry": "fa_prepare_gqa_rope + fa_launch_prepared"}


def build_decode(ctx, rng, split=None):
    n, hq, hkv, D, ps = 64, 32, 8, 128, 16
    ctx_lens = rng.integers(512, 8193, n).astype(np.int32)
    pages_per = (ctx_lens + ps - 1) // ps
    total = int(pages_per.sum())
    ids = rng.permutation(total).astype(np.int32)
    bt = np.zeros((n, int(pages_per.max())), np.int32)
    cur = 0
    for s in range(n):
        bt[s, :pages_per[s]] = ids[cur:cur + pages_per[s]]
        cur += pages_per[s]
    width = hkv * D
    kp = fa.DeviceBuffer.from_array(ctx, bf16_normal(rng, total * ps * width))
    vp = fa.DeviceBuffer.from_array(ctx, bf16_normal(rng, total * ps * width))
    q = fa.DeviceBuffer.from_array(ctx, bf16_normal(rng, n * hq * D))
    plan = fa.PagedDecodePlan(ctx, bt, ctx_lens, ps, total, hq, hkv, D,
                              fa.FlatAttentionConfig(True), 10000.0, fa.DTYPE_BF16)
    if split:
        plan.set_split(split)
    out = fa.DeviceBuffer(ctx, plan.layout().combined_bytes)
    # prepare cost: host work (work lists, validation, allocation) plus the stream-ordered
    # upload of the tables, until the stream has completed it; median of 5 after one warm-up
    prep_ms = []
    for _ in range(6):
        t0 = time.perf_counter()
        p2 = fa.PagedDecodePlan(ctx, bt, ctx_lens, ps, total, hq, hkv, D,
                                fa.FlatAttentionConfig(True), 10000.0, fa.DTYPE_BF16)
        ctx.synchronize()
        prep_ms.append((time.perf_counter() - t0) * 1e3)
        p2.release()
    # one serving step through the allocation-free entry point (work lists rebuilt on the host,
    # the stream-ordered metadata copy and the kernels) until the stream has completed it, the
    # Python call included; median of 10 after two warm-ups
    na_ms = []
    for _ in range(12):
        t0 = time.perf_counter()
        fa.paged_decode_noalloc(ctx, bt, ctx_lens, ps, total, hq, hkv, D,
                                fa.FlatAttentionConfig(True), 10000.0, fa.DTYPE_BF16, q, kp, vp,
                                out)
        ctx.synchronize()
        na_ms.append((time.perf_counter() - t0) * 1e3)
    nbytes = (float(ctx_lens.sum()) * hkv * D * 2 * 2 + n * hq * D * 2 * 2 + n * hq * 4
              + float(pages_per.sum()) * 4)
    run = lambda: plan.launch(q, kp, vp, out)  # noqa: E731
    info = plan.info()
    return run, nbytes, {"workload": "paged decode: 64 seqs ctx U[512,8192] page16 Hq32 Hkv8 "
                                     "D128 bf16 KV, shuffled pages",
                         "bytes_per_step": nbytes, "live_tokens": int(ctx_lens.sum()),
                         "prepare_ms": round(float(np.median(prep_ms[1:])), 4),
                         "noalloc_step_ms": round(float(np.median(na_ms[2:])), 4),
                         "split_tokens": info["split_tokens"], "work_items": info["work_items"]}


PEAK_F32_TFLOPS = 157.3    # MI355X dense fp32 matrix


def build_mha_f32(ctx, rng, causal, shape=(4, 16, 2048, 128)):
    """MHA B4 H16 N2048 D128, f32 I/O (configs[0] with shape=(1, 2, 128, 64))."""
    B, H, S, D = shape
    shape = fa.AttentionShape(B, H, S, D)
    ex = fa.HipFlatAttention(ctx)
    mk = lambda: fa.DeviceBuffer.from_array(ctx, rng.standard_normal(B * H * S * D, dtype=np.float32))  # noqa: E731
    q, k, v = mk(), mk(), mk()
    out = fa.DeviceBuffer(ctx, ex.layout(shape).combined_bytes)
    cfg = fa.FlatAttentionConfig(causal=causal)
    flop = 4.0 * B * H * D * (S * (S + 1) / 2 if causal else S * S)
    return (lambda: ex.forward_resident(q, k, v, shape, cfg, out)), flop


def build_chunked_paged(ctx, rng):
    """8 sequences x (2048 cached + 512 new) in a shuffled page-16 pool, Hq32 Hkv8
    D128 bf16, causal at offset 2048, RoPE theta 1e4 (K rotated on append). One step = the
    batched append of the 512 new tokens followed by the chunk's prefill over the paged cache."""
    n, hq, hkv, D, ps, cached, ql, theta = 8, 32, 8, 128, 16, 2048, 512, 1e4
    kv_len = cached + ql
    pages_per = kv_len // ps
    total = n * pages_per
    bt = rng.permutation(total).astype(np.int32).reshape(n, pages_per)
    width = hkv * D
    kp = fa.DeviceBuffer(ctx, total * ps * width * 2)
    vp = fa.DeviceBuffer(ctx, total * ps * width * 2)
    rot = fa.RotaryEmbeddingConfig(theta, 0)
    fa.paged_append_batched(ctx, bt, np.zeros(n, np.int32), cached, ps, total, hkv, D,
                            fa.DeviceBuffer.from_array(ctx, bf16_normal(rng, n * cached * width)),
                            fa.DeviceBuffer.from_array(ctx, bf16_normal(rng, n * cached * width)),
                            kp, vp, rot, fa.DTYPE_BF16)
    new_k = fa.DeviceBuffer.from_array(ctx, bf16_normal(rng, n * ql * width))
    new_v = fa.DeviceBuffer.from_array(ctx, bf16_normal(rng, n * ql * width))
    starts = np.full(n, cached, np.int32)
    shape = fa.AsymmetricGroupedAttentionShape(n, hq, hkv, ql, kv_len, D, cached)
    plan = fa.PagedChunkedPrefillPlan(ctx, bt, ps, total, shape, fa.FlatAttentionConfig(True),
                                      fa.AsymmetricRotaryEmbeddingConfig(theta, cached, 0),
                                      fa.DTYPE_BF16)
    q = fa.DeviceBuffer.from_array(ctx, bf16_normal(rng, n * ql * hq * D))
    out = fa.DeviceBuffer(ctx, plan.layout().combined_bytes)

    def append():
        fa.paged_append_batched(ctx, bt, starts, ql, ps, total, hkv, D, new_k, new_v, kp, vp,
                                rot, fa.DTYPE_BF16)

    flop = 4.0 * n * hq * D * (ql * cached + ql * (ql + 1) / 2)
    append_bytes = 2.0 * 2 * n * ql * width * 2  # K and V: read source, write pool
    return (lambda: plan.launch(q, kp, vp, out)), flop, append, append_bytes


def build_resident_decode(ctx, rng, dtype):
    """The reference's only published decode shape (M15/M48, docs/M48_THOR_REQUALIFICATION.md:69):
    B1 Hq16 Hkv4 D64 over 8192 resident rows (pre-rotated K), query at position 8191."""
    B, hq, hkv, D, cap = 1, 16, 4, 64, 8192
    width = hkv * D
    if dtype == fa.DTYPE_F32:
        mk = lambda n: rng.standard_normal(n, dtype=np.float32)  # noqa: E731
    else:
        mk = lambda n: bf16_normal(rng, n)  # noqa: E731
    k = fa.DeviceBuffer.from_array(ctx, mk(B * cap * width))
    v = fa.DeviceBuffer.from_array(ctx, mk(B * cap * width))
    q = fa.DeviceBuffer.from_array(ctx, mk(B * hq * D))
    plan = fa.ResidentDecodePlan(ctx, B, cap, cap, hq, hkv, D, fa.FlatAttentionConfig(True), 1e4,
                                 cap - 1, dtype)
    out = fa.DeviceBuffer(ctx, plan.layout().combined_bytes)
    eb = 4 if dtype == fa.DTYPE_F32 else 2
    nbytes = 2.0 * B * cap * width * eb + B * hq * D * eb * 2 + B * hq * 4
    return (lambda: plan.launch(q, k, v, out)), nbytes


def build_m48_decode(ctx, rng, kv_len):
    """The M48 candidate (encode_pre_rotated_k_decode_kv_reuse src/wgpu_external_asymmetric.rs:216)
    at the published shape B1 Hq16 Hkv4 D64 f32 (docs/M48_THOR_REQUALIFICATION.md:65-69): one
    call validates, builds the one-page-per-sequence plan, launches and releases it."""
    B, hq, hkv, D = 1, 16, 4, 64
    width = hkv * D
    mk = lambda n: rng.standard_normal(n, dtype=np.float32)  # noqa: E731
    k = fa.DeviceBuffer.from_array(ctx, mk(B * kv_len * width))
    v = fa.DeviceBuffer.from_array(ctx, mk(B * kv_len * width))
    q = fa.DeviceBuffer.from_array(ctx, mk(B * hq * D))
    shape = fa.AsymmetricGroupedAttentionShape(B, hq, hkv, 1, kv_len, D, kv_len - 1)
    rot = fa.AsymmetricRotaryEmbeddingConfig(1e4, kv_len - 1, 0)
    pipe = fa.HipAsymmetricProjectionPipeline.with_decode_kv_reuse(ctx, True)
    out = pipe.create_output_buffer(shape)
    cfg = fa.FlatAttentionConfig(True)
    nbytes = 2.0 * B * kv_len * width * 4 + B * hq * D * 4 * 2 + B * hq * 4
    return (lambda: pipe.encode_pre_rotated_k_decode_kv_reuse(q, k, v, out, shape, cfg, rot)), nbytes


def build_backward(ctx, rng, S=4096, data="normal"):
    """Recompute backward (dQ, dK, dV) at the prefill's shape without RoPE (the reference's
    backward has none): causal GQA B2 Hq32 Hkv8 D128 bf16. Algorithmic work: the five
    S x S x D products of attention backward (Q K^T, dO V^T, P^T dO, dS^T Q, dS K), i.e. 2.5x
    the forward's FLOPs; the kernels recompute Q K^T and dO V^T once more for dQ."""
    B, hq, hkv, D = 2, 32, 8, 128
    shape = fa.GroupedAttentionShape(B, hq, hkv, S, D)
    pipe = fa.HipGroupedBackwardRecomputePipeline(ctx, fa.DTYPE_BF16)
    lay = pipe.layout(shape)
    fwd = fa.DeviceBuffer(ctx, lay.packed_forward_bytes)
    nq, nkv = lay.q_elements, lay.kv_elements
    for off, n in ((lay.q_offset, nq), (lay.k_offset, nkv), (lay.v_offset, nkv),
                   (lay.d_out_offset, nq)):
        fwd.upload(bf16_normal(rng, n) if data == "normal"
                   else fa.f32_to_bf16_bits(np.full(n, 0.5, np.float32)), off)
    cfg = fa.FlatAttentionConfig(causal=True)
    # O and LSE from this library's forward over the same Q, K, V
    ex = fa.HipRotaryGroupedAttention(ctx, fa.DTYPE_BF16)
    flay = ex.layout(shape)
    out = fa.DeviceBuffer(ctx, flay.combined_bytes)
    view = lambda off, n: fa.DeviceBuffer(ctx, n, fwd.ptr + off)  # noqa: E731
    ex.forward_resident(view(lay.q_offset, nq * 2), view(lay.k_offset, nkv * 2),
                        view(lay.v_offset, nkv * 2), shape, cfg, None, out)
    ctx.synchronize()
    ev = HipEvents()
    ev.copy_d2d(fwd.ptr + lay.output_offset, out.ptr, nq * 2, ctx.stream)
    ev.copy_d2d(fwd.ptr + lay.lse_offset, out.ptr + flay.lse_byte_offset, lay.lse_elements * 4,
                ctx.stream)
    ctx.synchronize()
    out.free()
    grads = pipe.create_gradient_buffer(shape)
    prep = pipe.prepare(fwd, grads, shape, cfg)
    flop = 10.0 * B * hq * D * S * (S + 1) / 2
    return (lambda: pipe.encode_prepared(prep)), flop


def measure_backward(ctx, rng, steps, warmup, data="normal"):
    """`--only backward`: the recompute backward alone, op time from HIP events on the library's
    stream and the three kernels' time from the library's per-dispatch events, in one pass."""
    run, flop = build_backward(ctx, rng, data=data)
    ev = HipEvents()
    for _ in range(warmup):
        run()
    tel = ctx.last_telemetry()
    ctx.synchronize()
    op_ms = alternate_timing(ctx, ev, run, steps)
    total, cnt = ctx.kernel_timing(tel.kernel_id)
    ctx.set_kernel_timing(False)
    k_ms = total / max(cnt, 1)
    tf, ktf = flop / (op_ms * 1e-3) / 1e12, flop / (k_ms * 1e-3) / 1e12
    return {"metric": "recompute backward (dQ, dK, dV) TFLOP/s, causal GQA D128 N4096",
            "value": round(tf, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": steps,
            "warmup": warmup, "ms_per_step": round(op_ms, 4), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic" if data == "normal" else
                    "synthetic constant 0.5 (power-limit diagnostic, not the benchmark)",
            "config": {"workload": "recompute backward: causal GQA B2 Hq32 Hkv8 N4096 D128 bf16",
                       "flop_per_step": flop, "parallelism": "single GPU"},
            "kernel": tel.kernel_name, "kernel_ms": round(k_ms, 4),
            "roofline": {"bound": "mfma", "achieved": round(ktf, 2), "peak": PEAK_BF16_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(ktf / PEAK_BF16_TFLOPS, 4),
                         "traffic": None}}


def alternate_timing(ctx, ev, run, steps):
    """`steps` calls of `run` in one pass: odd calls bracketed by HIP events only (op time),
    even calls with the library's per-dispatch events too (kernel times). Returns the mean op
    time in ms; the kernel totals stay in the context."""
    evs = [(ev.create(), ev.create()) for _ in range(steps)]
    ctx.set_kernel_timing(True)
    for s in range(steps):
        ctx.pause_kernel_timing(s % 2 == 1)
        ev.record(evs[s][0], ctx.stream)
        run()
        ev.record(evs[s][1], ctx.stream)
    ctx.pause_kernel_timing(False)
    ctx.synchronize()
    op_steps = [s for s in range(steps) if s % 2 == 1] or list(range(steps))
    return float(np.mean([ev.elapsed_ms(*evs[s]) for s in op_steps]))


def graph_replay_ms(ctx, ev, run, steps=20):
    """Median op time of `run` captured once into a HIP graph (fa_graph_*) and replayed:
    HIP events around each replay on the library's stream, after five untimed replays."""
    run()  # the context's caches are sized before the capture
    with ctx.capture() as cap:
        run()
    for _ in range(5):
        cap.graph.launch()
    evs = [(ev.create(), ev.create()) for _ in range(steps)]
    for e0, e1 in evs:
        ev.record(e0, ctx.stream)
        cap.graph.launch()
        ev.record(e1, ctx.stream)
    ctx.synchronize()
    ms = float(np.median([ev.elapsed_ms(e0, e1) for e0, e1 in evs]))
    cap.graph.release()
    return ms


def _rec(kernel, op_ms, k_ms, work, bound, peak, unit, traffic=None, **extra):
    """A sub-record: op and kernel times, the rate over the whole op and the kernel's roofline."""
    rate_op = work / (op_ms * 1e-3) / (1e12 if unit == "TFLOP/s" else 1e9)
    rate_k = work / (k_ms * 1e-3) / (1e12 if unit == "TFLOP/s" else 1e9)
    return {"kernel": kernel, "ms": round(op_ms, 5), "kernel_ms": round(k_ms, 5),
            unit: round(rate_op, 2),
            "roofline": {"bound": bound, "achieved": round(rate_k, 2), "peak": peak,
                         "unit": unit, "frac": round(rate_k / peak, 4), "traffic": traffic},
            **extra}


def measure_baseline_configs(ctx, ev, rng, steps, with_cpu, warm=100):
    """Every other BASELINE config (and the two alternative cfg3 prefill kernels), each timed
    alone after `warm` untimed calls: op time from HIP events, the dominant kernel's time from
    the library's per-dispatch events, a roofline, and the CPU oracle timed on a bounded sample
    of the same workload (single core)."""
    res = {}

    def timed(run):
        for _ in range(warm):
            run()
        tel = ctx.last_telemetry()
        ctx.synchronize()
        op_ms = alternate_timing(ctx, ev, run, steps)
        total, cnt = ctx.kernel_timing(tel.kernel_id)
        ctx.set_kernel_timing(False)
        return op_ms, total / max(cnt, 1), tel

    cpu = cpu_baseline_configs() if with_cpu else {}
    # the reference's CPU-runnable case (MHA B1 H2 N128 D64 causal f32)
    run, flop = build_mha_f32(ctx, rng, True, shape=(1, 2, 128, 64))
    op_ms, k_ms, tel = timed(run)
    res["cfg1_mha_f32_causal_B1_H2_N128_D64"] = _rec(
        tel.kernel_name, op_ms, k_ms, flop, "mfma", PEAK_F32_TFLOPS, "TFLOP/s",
        note="launch-bound: 4.2 MFLOP", cpu_baseline=cpu.get("cfg1"))
    # MHA B4 H16 N2048 D128 f32, causal and non-causal
    for causal in (False, True):
        run, flop = build_mha_f32(ctx, rng, causal)
        op_ms, k_ms, tel = timed(run)
        key = "causal" if causal else "noncausal"
        res[f"cfg2_mha_f32_{key}_B4_H16_N2048_D128"] = _rec(
            tel.kernel_name, op_ms, k_ms, flop, "mfma", PEAK_F32_TFLOPS, "TFLOP/s",
            cpu_baseline=cpu.get(f"cfg2_{key}"))
    # configs[2] with the alternatives to the default prefill kernel
    ctx.set_prefill_precision(1)
    run, flop, _ = build_prefill(ctx, rng)
    op_ms, k_ms, tel = timed(run)
    res["cfg3_prefill_precise_scores"] = _rec(
        tel.kernel_name, op_ms, k_ms, flop, "mfma", PEAK_BF16_TFLOPS, "TFLOP/s",
        note="fa_ctx_set_prefill_precision(1): rotated Q and K carried as a 16-bit high part "
             "plus the residual, three Q.K^T MFMAs per k-step (f32-level scores; holds 2e-2 on "
             "the adversarial RoPE corpus)")
    ctx.set_prefill_precision(0)
    ctx.set_prefill_kernel(0)
    run, flop, _ = build_prefill(ctx, rng)
    op_ms, k_ms, tel = timed(run)
    res["cfg3_prefill_hip_main_loop"] = _rec(
        tel.kernel_name, op_ms, k_ms, flop, "mfma", PEAK_BF16_TFLOPS, "TFLOP/s",
        note="fa_ctx_set_prefill_kernel(0): the HIP main loop (8-wave ping-pong, 32 query rows "
             "per wave) instead of the default assembly kernel")
    ctx.set_prefill_kernel(-1)
    # chunked prefill into the paged cache (+ the batched append of the chunk)
    run, flop, append, append_bytes = build_chunked_paged(ctx, rng)
    op_ms, k_ms, tel = timed(run)
    res["cfg5_chunked_paged_prefill"] = _rec(
        tel.kernel_name, op_ms, k_ms, flop, "mfma", PEAK_BF16_TFLOPS, "TFLOP/s",
        cpu_baseline=cpu.get("cfg5"))
    op_ms, k_ms, tel = timed(append)
    res["cfg5_batched_append_512"] = _rec(tel.kernel_name, op_ms, k_ms, append_bytes, "hbm",
                                          PEAK_HBM_GBS, "GB/s")
    # the recompute backward at the prefill's shape (the reference's M18-M21 path)
    run, flop = build_backward(ctx, rng)
    op_ms, k_ms, tel = timed(run)
    res["backward_causal_gqa_B2_Hq32_Hkv8_N4096_D128_bf16"] = _rec(
        tel.kernel_name, op_ms, k_ms, flop, "mfma", PEAK_BF16_TFLOPS, "TFLOP/s",
        note="algorithmic FLOPs = 2.5x forward (five S x S x D products); kernel_ms spans the "
             "op's three launches (bwd_delta, the dK/dV kernel, bwd_dq_ds)", cpu_baseline=cpu.get("backward"))
    return res


def measure_all_configs(ctx, ev, rng, steps):
    """`--all-configs`: the reference's published decode shapes (M15 resident cache, M48), each
    timed alone (op events + its kernel's own events)."""
    stream = ctx.stream
    res = {}

    def timed(run):
        # warm up for 100 calls (clocks settle after tens of milliseconds of sustained work)
        for _ in range(100):
            run()
        tel = ctx.last_telemetry()
        ctx.synchronize()
        op_ms = alternate_timing(ctx, ev, run, steps)
        total, cnt = ctx.kernel_timing(tel.kernel_id)
        ctx.set_kernel_timing(False)
        return op_ms, total / max(cnt, 1), tel

    for dt, name in ((fa.DTYPE_F32, "f32"), (fa.DTYPE_BF16, "bf16")):
        run, nbytes = build_resident_decode(ctx, rng, dt)
        op_ms, k_ms, tel = timed(run)
        res[f"resident_decode_B1_Hq16_Hkv4_D64_kv8192_{name}"] = {
            "kernel": tel.kernel_name, "ms": round(op_ms, 4), "kernel_ms": round(k_ms, 4),
            "graph_ms": round(graph_replay_ms(ctx, ev, run), 4),
            "GB/s": round(nbytes / (k_ms * 1e-3) / 1e9, 1),
            "note": "one sequence: the op time is launch-bound, GB/s uses the kernel time",
            "reference_published_ms": {"M15": 23.843433, "M48": 19.562844,
                                       "hardware": "Jetson Thor, Vulkan, f32 (not comparable)"}}
    for kv_len, ref_ms in ((8192, 19.562844), (512, 1.317097)):
        run, nbytes = build_m48_decode(ctx, rng, kv_len)
        op_ms, k_ms, tel = timed(run)
        res[f"m48_decode_kv_reuse_B1_Hq16_Hkv4_D64_kv{kv_len}_f32"] = {
            "kernel": tel.kernel_name, "ms": round(op_ms, 4), "kernel_ms": round(k_ms, 4),
            "GB/s": round(nbytes / (k_ms * 1e-3) / 1e9, 1),
            "note": "ms includes the per-call plan (table upload, release waits for the stream)",
            "reference_published_ms": {"M48": ref_ms,
                                       "hardware": "Jetson Thor, Vulkan, f32 (not comparable)"}}
    return res


TRAFFIC_JSON = os.path.join(ROOT, "profiles", "hbm_traffic_prefill_decode.json")
COPY_BYTES = 1 << 30  # calibration copy: reads and writes exactly this many bytes


def summarize_pmc(fetch_csv: str, write_csv: str) -> dict:
    """HBM bytes per launch from two `rocprofv3 --pmc` runs of `bench.py --calibrate-copy`.

    FETCH_SIZE / WRITE_SIZE (KiB per dispatch) are scaled by what the same counter reads for
    the calibration copy of COPY_BYTES, so that the copy counts exactly COPY_BYTES each way."""
    import collections
    import csv

    def load(path, counter):
        per = collections.defaultdict(list)
        for r in csv.DictReader(open(path)):
            if r["Counter_Name"] == counter:
                per[r["Kernel_Name"]].append(float(r["Counter_Value"]))
        # median per kernel; for the copy kernel the largest dispatch is the calibration copy
        return {k: float(np.max(v) if "copyBuffer" in k else np.median(v)) for k, v in per.items()}

    fetch, write = load(fetch_csv, "FETCH_SIZE"), load(write_csv, "WRITE_SIZE")

    def pick(d, *keys):
        for k, v in d.items():
            if all(x in k for x in keys):
                return v
        raise KeyError(keys)

    copy_f = pick(fetch, "copyBuffer") * 1024.0
    copy_w = pick(write, "copyBuffer") * 1024.0
    f_scale, w_scale = COPY_BYTES / copy_f, COPY_BYTES / copy_w
    res = {"copy_bytes": COPY_BYTES, "fetch_scale": f_scale, "write_scale": w_scale}
    for name, key in (("prefill", "prefill_a64"), ("prefill_hip", "prefill_mfma16"),
                      ("decode", "decode_mfma"),
                      ("combine", "decode_combine"), ("rotate", "rotate_rows"),
                      ("bwd_delta", "bwd_delta<"), ("bwd_dkdv_a64", "bwd_dkdv_a64"),
                      ("bwd_dkdv", "bwd_dkdv<"),
                      ("bwd_dq_ds", "bwd_dq_ds<"), ("bwd_dq", "bwd_dq<")):
        try:
            fb = pick(fetch, key) * 1024.0 * f_scale
            wb = pick(write, key) * 1024.0 * w_scale
        except KeyError:
            continue
        res[name] = {"fetch_bytes": fb, "write_bytes": wb, "traffic_bytes": fb + wb,
                     "raw_fetch_kib": fb / 1024.0 / f_scale, "raw_write_kib": wb / 1024.0 / w_scale}
    return res


def load_traffic():
    try:
        return json.load(open(TRAFFIC_JSON))
    except (OSError, ValueError):
        return None


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cpu_threads() -> int:
    """Worker threads for the all-core leg: the host cores this process may use, at most 16
    (one GPU's share of the box)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def _timed_samples(fn, samples: int) -> dict:
    """One untimed warm-up call, then `samples` timed calls (wall clock, output allocation
    included as in examples/m28_scalar_flat_baseline.rs:100-179): median and p95 seconds."""
    fn()
    ts = []
    for _ in range(samples):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return {"median_s": float(np.median(ts)), "p95_s": float(np.percentile(ts, 95)),
            "samples": samples}


def cpu_baseline(samples: int = 5):
    """Scalar C oracle (oracle/) timed on this host on bounded samples of the same workloads,
    single-threaded and over all cores (independent (batch, head) units / sequences per
    thread). Rates use the median sample; p95 is reported beside it."""
    import oracle  # CPU baseline leg only
    threads = _cpu_threads()
    model = _cpu_model()
    res = {}
    # prefill: (b, h) units of configs[2] truncated to their first n query rows (causal rows
    # 0..n-1 do the same work as in the full problem); FLOP counted like the GPU metric.
    n, D, theta = 1024, 128, 10000.0
    flop_unit = 4.0 * D * n * (n + 1) / 2
    q = oracle.fill_normal(threads * n * D, 1)
    k = oracle.fill_normal(threads * n * D, 2)
    v = oracle.fill_normal(threads * n * D, 3)
    one = _timed_samples(lambda: oracle.forward_grouped_rope(
        q[:n * D], k[:n * D], v[:n * D], 1, 1, 1, n, D, True, theta, 0), samples)
    allc = _timed_samples(lambda: oracle.forward_grouped_rope(
        q, k, v, 1, threads, threads, n, D, True, theta, 0, threads=threads), samples)
    res["prefill"] = {
        "value": flop_unit / one["median_s"] / 1e12, "unit": "TFLOP/s", "cores": 1,
        "kind": "port", "p95_value": flop_unit / one["p95_s"] / 1e12,
        "sample": f"oracle forward_reference_grouped_rope (RoPE theta 1e4, D128, causal), one "
                  f"(b,h) unit of configs[2], its first {n} query rows; median of {samples} "
                  f"after a warm-up ({one['median_s']:.2f} s, p95 {one['p95_s']:.2f} s)",
        "all_cores": {"value": threads * flop_unit / allc["median_s"] / 1e12,
                      "p95_value": threads * flop_unit / allc["p95_s"] / 1e12,
                      "cores": threads, "sample": f"{threads} such units, one per thread "
                      f"({allc['median_s']:.2f} s median)"},
        "cpu_model": model}
    # decode: sequences of 4096 live tokens, Hq32 Hkv8 D128. The oracle reads f32 pools, so the
    # bytes are counted at 4 per element (every live K/V element once, plus Q, O, LSE, tables).
    ctxl, hq, hkv, ps = 4096, 32, 8, 16
    ns = 2 * threads
    pages = ctxl // ps
    bt = np.arange(ns * pages, dtype=np.int32).reshape(ns, pages)
    kp = oracle.fill_normal(ns * ctxl * hkv * D, 4)
    vp = oracle.fill_normal(ns * ctxl * hkv * D, 5)
    qd = oracle.fill_normal(ns * hq * D, 6)

    def nbytes(m):
        return m * (ctxl * hkv * D * 2 * 4 + hq * D * 4 * 2 + hq * 4 + pages * 4)

    n1 = 4
    one = _timed_samples(lambda: oracle.paged_decode(
        qd[:n1 * hq * D], kp, vp, ns * pages, ps, bt[:n1], [ctxl] * n1, hq, hkv, D, True, theta),
        samples)
    allc = _timed_samples(lambda: oracle.paged_decode(
        qd, kp, vp, ns * pages, ps, bt, [ctxl] * ns, hq, hkv, D, True, theta, threads=threads),
        samples)
    res["decode"] = {
        "value": nbytes(n1) / one["median_s"] / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
        "p95_value": nbytes(n1) / one["p95_s"] / 1e9,
        "sample": f"oracle paged decode, {n1} seqs x {ctxl} tokens, Hq32 Hkv8 D128, f32 pools "
                  f"(4 B per element); median of {samples} after a warm-up "
                  f"({one['median_s']:.2f} s, p95 {one['p95_s']:.2f} s)",
        "all_cores": {"value": nbytes(ns) / allc["median_s"] / 1e9,
                      "p95_value": nbytes(ns) / allc["p95_s"] / 1e9, "cores": threads,
                      "sample": f"{ns} seqs over {threads} threads "
                                f"({allc['median_s']:.2f} s median)"},
        "cpu_model": model}
    return res


def cpu_baseline_configs(samples: int = 3) -> dict:
    """Single-core C oracle on bounded samples of configs[0], [1], [4] and the backward: the
    whole of configs[0]; one (b, h) unit of configs[1] truncated to its first 1024 query rows
    (and, non-causal, 1024 keys); one (sequence, query head) of configs[4]; one (b, kv head)
    unit of the backward truncated to 1024 rows. FLOPs counted like the GPU figures."""
    import oracle  # CPU baseline leg only
    res = {}

    def rec(flop, fn, sample):
        t = _timed_samples(fn, samples)
        return {"value": flop / t["median_s"] / 1e12, "unit": "TFLOP/s", "cores": 1,
                "kind": "port", "p95_value": flop / t["p95_s"] / 1e12,
                "sample": f"{sample}; median of {samples} after a warm-up "
                          f"({t['median_s']:.3f} s)"}

    n, D = 128, 64
    q, k, v = (oracle.fill_normal(2 * n * D, s) for s in (21, 22, 23))
    res["cfg1"] = rec(4.0 * 2 * D * n * (n + 1) / 2,
                      lambda: oracle.forward(q, k, v, 1, 2, n, D, True),
                      "oracle forward_reference, the whole of configs[0]")
    n, D = 1024, 128
    q, k, v = (oracle.fill_normal(n * D, s) for s in (24, 25, 26))
    res["cfg2_causal"] = rec(4.0 * D * n * (n + 1) / 2,
                             lambda: oracle.forward(q, k, v, 1, 1, n, D, True),
                             f"oracle forward_reference f32, one (b,h) unit, {n} rows causal")
    res["cfg2_noncausal"] = rec(4.0 * D * n * n,
                                lambda: oracle.forward(q, k, v, 1, 1, n, D, False),
                                f"oracle forward_reference f32, one (b,h) unit, {n}x{n} keys")
    ql, kvl, off = 512, 2560, 2048
    q5 = oracle.fill_normal(ql * D, 27)
    k5, v5 = oracle.fill_normal(kvl * D, 28), oracle.fill_normal(kvl * D, 29)
    res["cfg5"] = rec(4.0 * D * (ql * off + ql * (ql + 1) / 2),
                      lambda: oracle.forward_projection_asymmetric(
                          q5, k5, v5, 1, 1, 1, ql, kvl, D, off, True, 1e4, off, 0, False),
                      "oracle asymmetric projection forward (pre-rotated K), one sequence and "
                      "query head of configs[4]: 512 new rows over 2560 keys")
    n, G = 1024, 4
    qb, kb, vb, dob = (oracle.fill_normal(m * n * D, s)
                       for m, s in ((G, 31), (1, 32), (1, 33), (G, 34)))
    o, lse = oracle.forward_grouped(qb, kb, vb, 1, G, 1, n, D, True)
    res["backward"] = rec(10.0 * G * D * n * (n + 1) / 2,
                          lambda: oracle.backward_grouped(qb, kb, vb, dob, o, lse, 1, G, 1, n, D,
                                                          True),
                          f"oracle backward_reference_grouped, one (b, kv head) unit with its {G} "
                          f"query heads, causal, first {n} rows")
    return res


def cpu_baseline_backward():
    """Scalar C oracle of the recompute backward (oracle/, backward_reference_grouped) on one
    (batch, kv head) unit of the backward workload: its 4 query heads, causal, N = 4096 rows
    (about 10 s on one core)."""
    import oracle  # CPU baseline leg only
    n, D, G = 4096, 128, 4
    q = oracle.fill_normal(G * n * D, 11)
    k = oracle.fill_normal(n * D, 12)
    v = oracle.fill_normal(n * D, 13)
    do = oracle.fill_normal(G * n * D, 14)
    o, lse = oracle.forward_grouped(q, k, v, 1, G, 1, n, D, True)
    t0 = time.perf_counter()
    oracle.backward_grouped(q, k, v, do, o, lse, 1, G, 1, n, D, True)
    dt = time.perf_counter() - t0
    flop = 10.0 * G * D * n * (n + 1) / 2
    return {"value": flop / dt / 1e12, "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": f"oracle backward_reference_grouped, one (b, kv head) unit with its {G} "
                      f"query heads, causal N={n}, D{D}, {dt:.2f} s"}


def _traffic(traffic, name):
    """HBM bytes per launch of the op's dominant kernel, from the committed PMC summary."""
    if not traffic or name not in traffic:
        return None
    return round(traffic[name]["traffic_bytes"])


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # The GPU's clocks take a few tens of milliseconds of sustained work to settle: 200 untimed
    # steps (~0.1 s) precede 100 timed ones, so the figures are steady-state throughput.
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="skip the other BASELINE configs (configs[0], [1], [4], backward, and "
                         "the alternative cfg3 prefill kernels)")
    ap.add_argument("--prefill-kernel", type=int, default=-1,
                    help="-1 auto (assembly main loop where it applies), 0 HIP kernels only "
                         "(fa_ctx_set_prefill_kernel)")
    ap.add_argument("--prefill-policy", type=int, default=-1,
                    help="-1 auto, 0 rotate K on load, 1 pre-rotate K")
    ap.add_argument("--only", choices=["prefill", "decode", "backward"], default=None,
                    help="time one op alone (backward: the recompute backward at the prefill "
                         "shape, a line of its own)")
    ap.add_argument("--backward-kernel", type=int, default=-1,
                    help="--only backward: -1 / 1 the assembly dK/dV kernel where it applies "
                         "(default), 0 the HIP kernel (fa_ctx_set_backward_kernel)")
    ap.add_argument("--backward-policy", type=int, default=-1,
                    help="--only backward: -1 stored dS (default), 0 dQ recomputes S and dP "
                         "(fa_ctx_set_backward_policy)")
    ap.add_argument("--decode-split", type=int, default=None,
                    help="tokens per split-K partition of the decode plan (default: automatic)")
    ap.add_argument("--all-configs", action="store_true",
                    help="also time the reference's published decode shapes (M15, M48)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run one device copy of 1 GiB (counter calibration for --pmc runs)")
    ap.add_argument("--data", choices=["normal", "constant"], default="normal",
                    help="prefill and backward inputs: N(0,1) (the benchmark), or a constant 0.5 everywhere "
                         "(power-limit diagnostic; not a benchmark figure)")
    ap.add_argument("--ceilings", action="store_true",
                    help="print the practical ceilings instead: a pure bf16 MFMA stream on random "
                         "and constant operands, streaming HBM reads at 4 / 8 / 16 loads in flight")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="turn two rocprofv3 --pmc counter CSVs into the traffic summary")
    ap.add_argument("--traffic-out", default=TRAFFIC_JSON,
                    help="where --summarize-pmc writes (default: the prefill/decode summary that "
                         "the bench line's roofline.traffic reads)")
    args = ap.parse_args()
    if args.summarize_pmc:
        res = summarize_pmc(*args.summarize_pmc)
        os.makedirs(os.path.dirname(os.path.abspath(args.traffic_out)), exist_ok=True)
        with open(args.traffic_out, "w") as f:
            json.dump(res, f, indent=1)
        print(json.dumps(res))
        return
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (each GPU would "
              "run its own shard of sequences / heads; nothing crosses GPUs on this path)",
              file=sys.stderr)
        sys.exit(2)

    if args.ceilings:
        from flat_attention_amd import diag
        res = {"mfma_bf16_tflops": {"random": round(diag.mfma_ceiling(0, False), 1),
                                    "constant": round(diag.mfma_ceiling(0, True), 1),
                                    "spec": PEAK_BF16_TFLOPS},
               "mfma_f32_tflops": {"random": round(diag.mfma_ceiling(0, False, diag.DTYPE_F32), 1),
                                   "constant": round(diag.mfma_ceiling(0, True, diag.DTYPE_F32), 1),
                                   "spec": PEAK_F32_TFLOPS},
               "stream_read_tbps": {str(d): round(diag.stream_read(0, d), 3) for d in (4, 8, 16)},
               "hbm_spec_tbps": PEAK_HBM_GBS / 1000.0}
        print(json.dumps(res))
        return
    rng = np.random.default_rng(1234)
    ctx = fa.HipContext(0)
    if args.only == "backward":
        ctx.set_backward_policy(args.backward_policy)
        ctx.set_backward_kernel(args.backward_kernel)
        out = measure_backward(ctx, rng, args.steps, args.warmup, args.data)
        if args.calibrate_copy:
            a, b = fa.DeviceBuffer(ctx, COPY_BYTES), fa.DeviceBuffer(ctx, COPY_BYTES)
            HipEvents().copy_d2d(b.ptr, a.ptr, COPY_BYTES, ctx.stream)
            ctx.synchronize()
            a.free()
            b.free()
        if not args.no_cpu_baseline:
            out["cpu_baseline"] = cpu_baseline_backward()
        print(json.dumps(out))
        ctx.close()
        return
    ev = HipEvents()
    stream = ctx.stream
    ctx.set_prefill_policy(args.prefill_policy)
    ctx.set_prefill_kernel(args.prefill_kernel)
    ops = []
    if args.only in (None, "prefill"):
        ops.append(("prefill",) + build_prefill(ctx, rng, args.data))
    if args.only in (None, "decode"):
        ops.append(("decode",) + build_decode(ctx, rng, args.decode_split))
    ctx.synchronize()
    # The other BASELINE configs are measured next (each after its own warm-up, inputs built
    # beforehand): the headline's warm-up and timed steps then run right after sustained GPU
    # work, not after the host-side set-up that leaves the GPU idle (a power-management dip of
    # ~30 calls follows an idle GPU).
    baseline_configs = None
    if args.only is None and not args.no_other_configs and args.data == "normal":
        baseline_configs = measure_baseline_configs(ctx, ev, rng, max(args.steps // 2, 10),
                                                    not args.no_cpu_baseline)
        ctx.set_prefill_policy(args.prefill_policy)
        ctx.set_prefill_kernel(args.prefill_kernel)

    tele = {}
    for _ in range(args.warmup):
        for name, run, _, _ in ops:
            run()
            tele[name] = ctx.last_telemetry()
    ctx.synchronize()

    # One timed pass of alternating steps: odd steps carry only HIP events around each op on
    # the library's stream (the op times), even steps also the library's own per-dispatch
    # events around every kernel (fa_ctx_set_kernel_timing; they add a few µs between kernels,
    # so they stay out of the op times). Both describe the same run at the same clocks.
    evs = [[ev.create() for _ in range(len(ops) + 1)] for _ in range(args.steps)]
    ctx.set_kernel_timing(True)
    t_wall = time.perf_counter()
    for s in range(args.steps):
        ctx.pause_kernel_timing(s % 2 == 1)
        ev.record(evs[s][0], stream)
        for i, (name, run, _, _) in enumerate(ops):
            run()
            ev.record(evs[s][i + 1], stream)
            if s == 0:
                tele[name] = ctx.last_telemetry()
    ctx.synchronize()
    wall = time.perf_counter() - t_wall
    kern, kern_min = {}, {}
    for name, _, _, _ in ops:
        total, n = ctx.kernel_timing(tele[name].kernel_id)
        kern[name] = total / max(n, 1)
        kern_min[name] = ctx.kernel_timing_range(tele[name].kernel_id)[0]
    ctx.set_kernel_timing(False)
    if args.calibrate_copy:
        a, b = fa.DeviceBuffer(ctx, COPY_BYTES), fa.DeviceBuffer(ctx, COPY_BYTES)
        ev.copy_d2d(b.ptr, a.ptr, COPY_BYTES, stream)
        ctx.synchronize()
        a.free()
        b.free()
    op_steps = [s for s in range(args.steps) if s % 2 == 1] or list(range(args.steps))
    per_op = {name: [ev.elapsed_ms(evs[s][i], evs[s][i + 1]) for s in op_steps]
              for i, (name, _, _, _) in enumerate(ops)}
    # the same ops replayed from a captured HIP graph (launch overhead removed), after the
    # timed pass; reported beside the op times, not used for `value`
    graph_ms = {name: graph_replay_ms(ctx, ev, run) for name, run, _, _ in ops}
    step_ms = sum(np.mean(v) for v in per_op.values())

    out = {"metric": "causal GQA prefill TFLOP/s (D128,N4096) + paged-decode HBM GB/s, % of peak",
           "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": round(step_ms, 4), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "bf16",
           "data": "synthetic" if args.data == "normal" else
                   "synthetic constant 0.5 (power-limit diagnostic, not the benchmark)",
           "wall_s": round(wall, 3)}
    details = {}
    traffic = load_traffic()
    for name, run, work, meta in ops:
        ms = float(np.mean(per_op[name]))
        t = tele[name]
        d = {"ms": round(ms, 5), "ms_min": round(float(np.min(per_op[name])), 5),
             "kernel": t.kernel_name, "kernel_id": t.kernel_id, "dispatches": t.dispatch_count,
             "grid": list(t.workgroups), **meta}
        d["kernel_ms"] = round(kern[name], 5)
        d["kernel_ms_min"] = round(kern_min[name], 5)
        d["graph_ms"] = round(graph_ms[name], 5)
        if name == "prefill":
            tf = work / (ms * 1e-3) / 1e12
            ktf = work / (kern[name] * 1e-3) / 1e12
            d.update({"TFLOP/s": round(tf, 2),
                      "roofline": {"bound": "mfma", "achieved": round(ktf, 2),
                                   "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                                   "frac": round(ktf / PEAK_BF16_TFLOPS, 4),
                                   "traffic": _traffic(traffic, "prefill")}})
        else:
            gbs = work / (ms * 1e-3) / 1e9
            kgbs = work / (kern[name] * 1e-3) / 1e9
            d.update({"GB/s": round(gbs, 1),
                      "roofline": {"bound": "hbm", "achieved": round(kgbs, 1),
                                   "peak": PEAK_HBM_GBS, "unit": "GB/s",
                                   "frac": round(kgbs / PEAK_HBM_GBS, 4),
                                   "traffic": _traffic(traffic, "decode")}})
        details[name] = d
    if "prefill" in details:
        out["value"] = details["prefill"]["TFLOP/s"]
        out["unit"] = "TFLOP/s"
        out["roofline"] = details["prefill"]["roofline"]
    else:
        out["value"] = details["decode"]["GB/s"]
        out["unit"] = "GB/s"
        out["roofline"] = details["decode"]["roofline"]
    out["config"] = {"workload": " + ".join(d["workload"] for d in details.values()),
                     "configs": "BASELINE configs[2] (prefill) + configs[3] (decode)",
                     "parallelism": "single GPU"}
    out["prefill"] = details.get("prefill")
    out["decode"] = details.get("decode")
    # Steady-state check: the op times of the first and second halves of the timed steps. A
    # clock transient (a GPU that idled before the run) shows as a drift between the halves; a
    # kernel regression does not.
    head = "prefill" if "prefill" in details else "decode"
    v = per_op[head]
    h = max(len(v) // 2, 1)
    a, b = float(np.mean(v[:h])), float(np.mean(v[h:] or v))
    out["steady_state"] = {"op": head, "first_half_ms": round(a, 5), "second_half_ms": round(b, 5),
                           "drift": round(a / b - 1.0, 4), "steady": abs(a / b - 1.0) < 0.03,
                           "after_sustained_work": baseline_configs is not None}
    if not args.no_cpu_baseline:
        cb = cpu_baseline()
        primary = cb["prefill"] if "prefill" in details else cb["decode"]
        out["cpu_baseline"] = dict(primary, other=cb["decode"] if "prefill" in details else None)
    if baseline_configs is not None:
        out["other_configs"] = baseline_configs
    if args.all_configs:
        out["extra_configs"] = measure_all_configs(ctx, ev, rng, max(args.steps // 2, 5))
    ctx.close()
    print(json.dumps(out))


if __name__ == "__main__":
    main()
