"""Host-side checks of the C ABI that need no GPU: every symbol declared in include/flat_hip.h
is exported by the built library, the PagedKvTable restatement reproduces the reference's
known-answer tests (src/paged_kv.rs:196-271), and argument validation fails closed with the
reference's error variants before any device work (a null context is only reported once the
arguments are valid)."""
import ctypes
import os
import re

import numpy as np
import pytest

import flat_attention_amd as fa
from flat_attention_amd import _lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "flat_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fa_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = fa.lib()
    names = declared_functions()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) == set(L.PROTOTYPES), set(names) ^ set(L.PROTOTYPES)
    assert lib.fa_abi_version() == 1


def test_no_device_is_reported_as_unavailable_or_context_is_created():
    try:
        ctx = fa.HipContext(0)
    except fa.FlatHipError as e:
        assert e.variant == "Unavailable"
    else:
        ctx.close()


def test_resolved_scale_default_and_errors():
    assert fa.FlatAttentionConfig().resolved_scale(64) == 0.125  # src/lib.rs:527
    assert fa.FlatAttentionConfig(softmax_scale=0.5).resolved_scale(64) == 0.5
    for bad in (0.0, -1.0, float("inf"), float("nan")):
        with pytest.raises(fa.FlatHipError) as e:
            fa.FlatAttentionConfig(softmax_scale=bad).resolved_scale(64)
        assert e.value.variant == "InvalidScale"
    with pytest.raises(fa.FlatHipError) as e:
        fa.FlatAttentionConfig().resolved_scale(0)
    assert e.value.variant == "ZeroDimension"


def test_packed_layout():
    lay = fa.packed_layout(10, 3, fa.DTYPE_F32)
    assert (lay.output_bytes, lay.lse_byte_offset, lay.combined_bytes) == (40, 40, 52)
    lay = fa.packed_layout(5, 2, fa.DTYPE_BF16)  # odd 16-bit count: LSE aligned to 4 bytes
    assert (lay.output_bytes, lay.lse_byte_offset, lay.combined_bytes) == (10, 12, 20)


# --------------------------------------------------------------------------- PagedKvTable

def test_mapping_is_stable_across_page_boundaries():
    t = fa.PagedKvTable(fa.PagedKvConfig(4, 3))
    t.append(9)
    assert t.address(0).physical_page == 0
    assert t.address(3).offset_in_page == 3
    assert t.address(4).physical_page == 1
    assert t.address(8).physical_page == 2
    assert t.address(9) is None


def test_telemetry_reports_exact_internal_fragmentation():
    t = fa.PagedKvTable(fa.PagedKvConfig(8, 4))
    t.append(9)
    assert t.telemetry() == fa.PagedKvTelemetry(9, 32, 2, 2, 7, 0)


def test_reset_invalidates_old_generation_before_page_reuse():
    t = fa.PagedKvTable(fa.PagedKvConfig(2, 2))
    t.append(1)
    old = t.address(0)
    t.reset()
    assert t.address(0) is None
    t.append(1)
    new = t.address(0)
    assert old.physical_page == new.physical_page and old.generation != new.generation


def test_capacity_overflow_is_explicit_and_non_mutating():
    t = fa.PagedKvTable(fa.PagedKvConfig(4, 2))
    t.append(7)
    before = (len(t), t.telemetry(), t.block_row().tolist())
    with pytest.raises(fa.FlatHipError) as e:
        t.append(2)
    assert e.value.variant == "CapacityExceeded" and "requires 9 tokens, capacity is 8" in str(e.value)
    assert (len(t), t.telemetry(), t.block_row().tolist()) == before


def test_table_zero_dimension_and_block_row():
    with pytest.raises(fa.FlatHipError) as e:
        fa.PagedKvTable(fa.PagedKvConfig(0, 4))
    assert e.value.variant == "PagedZeroDimension"
    t = fa.PagedKvTable(fa.PagedKvConfig(3, 4))
    with pytest.raises(fa.FlatHipError) as e:
        t.block_row()
    assert e.value.variant == "EmptyTable"
    t.append(7)
    assert t.block_row().tolist() == [0, 1, 2]
    t.append(0)  # zero-token append is a no-op
    assert len(t) == 7
    c = t.clone()
    c.append(3)
    assert len(t) == 7 and len(c) == 10


# --------------------------------------------------------------------------- validation

FAKE = 0x1000  # non-null stand-in pointer: validation must fail before it is ever used


def _gqa(shape, cfg=None, rot=None, dtype=fa.DTYPE_F32, q_bytes=1 << 40, kv_bytes=1 << 40,
         out_bytes=1 << 40):
    cfg = cfg or fa.FlatAttentionConfig()
    r = ctypes.byref(rot.c()) if rot else None
    return fa.lib().fa_forward_gqa_rope(None, FAKE, q_bytes, FAKE, FAKE, kv_bytes, FAKE, out_bytes,
                                        ctypes.byref(shape.c()), ctypes.byref(cfg.c()), r, dtype)


def _variant(rc):
    return L.STATUS[rc]


def test_forward_validation_variants():
    g = fa.GroupedAttentionShape
    assert _variant(_gqa(g(0, 4, 2, 8, 64))) == "ZeroDimension"
    assert _variant(_gqa(g(1, 6, 4, 8, 64))) == "InvalidHeadGrouping"
    assert _variant(_gqa(g(1, 4, 2, 8, 256))) == "UnsupportedHeadDim"
    assert _variant(_gqa(g(1, 4, 2, 8, 60), dtype=fa.DTYPE_BF16)) == "UnsupportedHeadDim"
    assert _variant(_gqa(g(1, 4, 2, 8, 63), rot=fa.RotaryEmbeddingConfig(1e4))) == "InvalidRotaryHeadDim"
    assert _variant(_gqa(g(1, 4, 2, 8, 64), rot=fa.RotaryEmbeddingConfig(-1.0))) == "InvalidRotaryTheta"
    assert _variant(_gqa(g(1, 4, 2, 8, 64), rot=fa.RotaryEmbeddingConfig(1e4, 2**64 - 2))) == "PositionOverflow"
    assert _variant(_gqa(g(1, 4, 2, 8, 64), cfg=fa.FlatAttentionConfig(softmax_scale=0.0))) == "InvalidScale"
    assert _variant(_gqa(g(2**40, 2**20, 2**20, 2**10, 64))) == "ShapeOverflow"
    assert _variant(_gqa(g(1, 4, 2, 8, 64), q_bytes=100)) == "BufferTooSmall"
    assert _variant(_gqa(g(1, 4, 2, 8, 64), kv_bytes=100)) == "BufferTooSmall"
    assert _variant(_gqa(g(1, 4, 2, 8, 64), out_bytes=4 * 4 * 8 * 64)) == "BufferTooSmall"
    assert _variant(_gqa(g(1, 4, 2, 8, 64), dtype=7)) == "UnsupportedDtype"
    # valid arguments, no context: reported last
    assert _variant(_gqa(g(1, 4, 2, 8, 64))) == "NullArgument"
    msg = fa.lib().fa_last_error_message().decode()
    assert "context" in msg


def test_buffer_too_small_message_names_tensor_and_sizes():
    rc = _gqa(fa.GroupedAttentionShape(1, 4, 2, 8, 64), q_bytes=100)
    assert _variant(rc) == "BufferTooSmall"
    assert fa.lib().fa_last_error_message().decode() == \
        "buffer Q contains 100 bytes, requires at least 8192"


def test_chunked_prefill_zero_chunk_rejected():
    sh = fa.GroupedAttentionShape(1, 4, 2, 8, 64)
    rc = fa.lib().fa_chunked_prefill(None, FAKE, 1 << 30, FAKE, FAKE, 1 << 30, FAKE, 1 << 30,
                                     ctypes.byref(sh.c()),
                                     ctypes.byref(fa.FlatAttentionConfig(True).c()),
                                     ctypes.byref(fa.RotaryEmbeddingConfig(1e4).c()), 0,
                                     fa.DTYPE_F32)
    assert _variant(rc) == "ZeroQueryChunkSize"


def _decode_prepare(bt, lens, qpos=None, ps=16, pages=8, hq=4, hkv=2, D=64, theta=1e4,
                    causal=True, dtype=fa.DTYPE_F32):
    bt = np.ascontiguousarray(bt, np.int32)
    lens = np.ascontiguousarray(lens, np.int32)
    qp = None if qpos is None else np.ascontiguousarray(qpos, np.int32)
    h = L.VP()
    rc = fa.lib().fa_paged_decode_prepare(None, bt.ctypes.data, bt.shape[1], lens.ctypes.data,
                                          None if qp is None else qp.ctypes.data, lens.shape[0],
                                          ps, pages, hq, hkv, D,
                                          ctypes.byref(fa.FlatAttentionConfig(causal).c()), theta,
                                          dtype, ctypes.byref(h))
    return _variant(rc)


def test_decode_prepare_validation_variants():
    bt = [[0, 1, 2]]
    assert _decode_prepare(bt, [40], qpos=[20]) == "CausalVisibilityMismatch"
    assert _decode_prepare(bt, [40], qpos=[20], causal=False) == "NullArgument"
    assert _decode_prepare(bt, [0]) == "EmptyTable"
    assert _decode_prepare(bt, [49]) == "IndexSpaceExceeded"
    assert _decode_prepare([[0, 9, 1]], [40]) == "InvalidPage"
    assert _decode_prepare([[0, -1, 1]], [40]) == "InvalidPage"
    assert _decode_prepare(bt, [40], hq=6, hkv=4) == "InvalidHeadGrouping"
    assert _decode_prepare(bt, [40], D=256) == "UnsupportedHeadDim"
    assert _decode_prepare(bt, [40], D=66) == "UnsupportedHeadDim"
    assert _decode_prepare(bt, [40], D=63) == "InvalidRotaryHeadDim"
    assert _decode_prepare(bt, [40], theta=0.0) == "InvalidRotaryTheta"
    assert _decode_prepare(bt, [40], ps=0) == "PagedZeroDimension"
    assert _decode_prepare(bt, [40]) == "NullArgument"  # all valid, no context


def _decode_noalloc(bt, lens, qpos=None, ps=16, pages=8, hq=4, hkv=2, D=64, theta=1e4,
                    causal=True, dtype=fa.DTYPE_F32, q_bytes=None, pool_bytes=None,
                    out_bytes=None):
    """fa_paged_decode_noalloc with no context: every check before device work. The buffer
    arguments are stand-in addresses that are never dereferenced (the call stops at the null
    context, or earlier)."""
    bt = np.ascontiguousarray(bt, np.int32)
    lens = np.ascontiguousarray(lens, np.int32)
    qp = None if qpos is None else np.ascontiguousarray(qpos, np.int32)
    eb = 4 if dtype == fa.DTYPE_F32 else 2
    n = lens.shape[0]
    q_need = n * hq * D * eb
    pool_need = pages * ps * hkv * D * eb
    out_need = fa.packed_layout(n * hq * D, n * hq, dtype).combined_bytes
    fake = ctypes.c_void_p(0x1000)
    rc = fa.lib().fa_paged_decode_noalloc(
        None, bt.ctypes.data, bt.shape[1], lens.ctypes.data,
        None if qp is None else qp.ctypes.data, n, ps, pages, hq, hkv, D,
        ctypes.byref(fa.FlatAttentionConfig(causal).c()), theta, dtype,
        fake, q_need if q_bytes is None else q_bytes, fake, fake,
        pool_need if pool_bytes is None else pool_bytes, fake,
        out_need if out_bytes is None else out_bytes)
    return _variant(rc)


def test_noalloc_decode_validation_matches_prepare():
    """The allocation-free decode validates exactly as fa_paged_decode_prepare (shared checks),
    then its buffers, before it needs the context."""
    bt = [[0, 1, 2]]
    for kw in (dict(lens=[40], qpos=[20]), dict(lens=[0]), dict(lens=[49]),
               dict(lens=[40], hq=6, hkv=4), dict(lens=[40], D=256), dict(lens=[40], D=63),
               dict(lens=[40], theta=0.0), dict(lens=[40], ps=0)):
        lens = kw.pop("lens")
        assert _decode_noalloc(bt, lens, **kw) == _decode_prepare(bt, lens, **kw)
    assert _decode_noalloc([[0, 9, 1]], [40]) == "InvalidPage"
    assert _decode_noalloc(bt, [40], q_bytes=8) == "BufferTooSmall"
    assert _decode_noalloc(bt, [40], pool_bytes=8) == "BufferTooSmall"
    assert _decode_noalloc(bt, [40], out_bytes=8) == "BufferTooSmall"
    assert _decode_noalloc(bt, [40]) == "NullArgument"  # all valid, no context
    assert "context is null" in fa.lib().fa_last_error_message().decode()


def test_kernel_timing_calls_need_a_context():
    assert _variant(fa.lib().fa_ctx_pause_kernel_timing(None, 1)) == "NullArgument"
    assert _variant(fa.lib().fa_ctx_set_kernel_timing(None, 1)) == "NullArgument"


def _resident_prepare(batch=2, cap=64, kv_len=40, hq=4, hkv=2, D=64, theta=1e4, qpos=39,
                      causal=True, dtype=fa.DTYPE_F32):
    h = L.VP()
    rc = fa.lib().fa_resident_decode_prepare(None, batch, cap, kv_len, hq, hkv, D,
                                             ctypes.byref(fa.FlatAttentionConfig(causal).c()),
                                             theta, qpos, dtype, ctypes.byref(h))
    return _variant(rc)


def test_resident_decode_prepare_validation_variants():
    """ResidentDecodeError variants in the reference's check order (src/wgpu_decode.rs:419-510):
    causal visibility first, then zero dimensions, EmptyCache, InvalidCacheLength, head_dim,
    head grouping, theta; a null context is reported only once everything else is valid."""
    assert _resident_prepare(qpos=20) == "CausalVisibilityMismatch"
    assert _resident_prepare(qpos=20, causal=False) == "NullArgument"
    assert _resident_prepare(qpos=20, batch=0) == "CausalVisibilityMismatch"
    assert _resident_prepare(batch=0) == "ZeroDimension"
    assert _resident_prepare(cap=0, kv_len=0, qpos=0) == "ZeroDimension"
    assert _resident_prepare(kv_len=0, qpos=0) == "EmptyCache"
    assert _resident_prepare(kv_len=65, qpos=64) == "InvalidCacheLength"
    assert _resident_prepare(D=63) == "InvalidRotaryHeadDim"
    assert _resident_prepare(D=256) == "UnsupportedHeadDim"
    assert _resident_prepare(hq=6, hkv=4) == "InvalidHeadGrouping"
    assert _resident_prepare(theta=float("nan")) == "InvalidRotaryTheta"
    assert _resident_prepare() == "NullArgument"
    assert _resident_prepare(dtype=fa.DTYPE_BF16) == "NullArgument"


def _variable(meta, shape=(2, 4, 2, 8, 16, 64, 0), theta=1e4, kv_off=0, q_bytes=1 << 30):
    sh = fa.AsymmetricGroupedAttentionShape(*shape)
    arr = (L.VariableSequenceC * max(len(meta), 1))(*[L.VariableSequenceC(*m) for m in meta])
    return _variant(fa.lib().fa_forward_projection_variable(
        None, FAKE, q_bytes, FAKE, FAKE, 1 << 30, FAKE, 1 << 30, ctypes.byref(sh.c()), arr,
        len(meta), ctypes.byref(fa.FlatAttentionConfig(True).c()), theta, kv_off, fa.DTYPE_BF16))


def test_variable_prefill_validation_variants():
    """validate_dispatch src/wgpu_external_variable.rs:229, in its order; a null context is
    reported last."""
    ok = [(8, 16, 0, 0), (3, 5, 2, 7)]
    assert _variable(ok[:1]) == "LengthMismatch"
    assert _variable([(0, 16, 0, 0), ok[1]]) == "ZeroDimension"
    assert _variable([(9, 16, 0, 0), ok[1]]) == "LengthMismatch"
    assert _variable([(8, 17, 0, 0), ok[1]]) == "LengthMismatch"
    assert _variable([(8, 16, 2**31 - 4, 0), ok[1]]) == "PositionOverflow"
    assert _variable([(8, 16, 0, 2**31 - 4), ok[1]]) == "PositionOverflow"
    assert _variable(ok, kv_off=2**31 - 8) == "PositionOverflow"
    assert _variable(ok, theta=0.0) == "InvalidRotaryTheta"
    assert _variable(ok, shape=(2, 4, 2, 8, 16, 63, 0)) == "InvalidRotaryHeadDim"
    assert _variable(ok, shape=(2, 6, 4, 8, 16, 64, 0)) == "InvalidHeadGrouping"
    assert _variable(ok, q_bytes=16) == "BufferTooSmall"
    assert _variable(ok) == "NullArgument"


def _kv_reuse(shape=(1, 16, 4, 1, 192, 64, 191), theta=1e4, q_rope=191, kv_rope=0,
              q_bytes=1 << 30, dtype=fa.DTYPE_F32, rotary=True):
    sh = fa.AsymmetricGroupedAttentionShape(*shape)
    rot = fa.AsymmetricRotaryEmbeddingConfig(theta, q_rope, kv_rope)
    return _variant(fa.lib().fa_forward_projection_asymmetric_decode_kv_reuse(
        None, FAKE, q_bytes, FAKE, FAKE, 1 << 30, FAKE, 1 << 30, ctypes.byref(sh.c()),
        ctypes.byref(fa.FlatAttentionConfig(True).c()),
        ctypes.byref(rot.c()) if rotary else None, dtype))


def test_decode_kv_reuse_validation_variants():
    """encode_pre_rotated_k_decode_kv_reuse src/wgpu_external_asymmetric.rs:216 in its order:
    shape validation (tests/m48_decode_kv_reuse.rs:267: zero KV heads is ZeroDimension), the
    candidate's query_len and group-size limits, then encode_with_options :291; a null context is
    reported last. Without the candidate the pipeline refuses (m48_is_opt_in :318)."""
    assert _kv_reuse(rotary=False) == "NullArgument"
    assert _kv_reuse(shape=(1, 16, 0, 1, 1, 64, 0), q_rope=0) == "ZeroDimension"
    assert _kv_reuse(shape=(1, 16, 5, 1, 8, 64, 7)) == "InvalidHeadGrouping"
    assert _kv_reuse(shape=(1, 16, 4, 2, 8, 64, 7)) == "UnsupportedCandidateShape"
    assert _kv_reuse(shape=(1, 4, 4, 1, 8, 64, 7)) == "UnsupportedCandidateShape"
    assert _kv_reuse(shape=(1, 16, 4, 1, 8, 64, 2**31 - 1)) == "PositionOverflow"
    assert _kv_reuse(q_rope=2**31) == "PositionOverflow"
    assert _kv_reuse(theta=-1.0) == "InvalidRotaryTheta"
    assert _kv_reuse(shape=(1, 16, 4, 1, 8, 63, 7)) == "InvalidRotaryHeadDim"
    assert _kv_reuse(shape=(1, 16, 4, 1, 8, 132, 7)) == "UnsupportedHeadDim"
    assert _kv_reuse(dtype=fa.DTYPE_BF16, shape=(1, 16, 4, 1, 8, 60, 7)) == "UnsupportedHeadDim"
    assert _kv_reuse(q_bytes=16) == "BufferTooSmall"
    assert _kv_reuse(dtype=9) == "UnsupportedDtype"
    assert _kv_reuse() == "NullArgument"
    assert _kv_reuse(shape=(1, 16, 4, 1, 8, 6, 7)) == "NullArgument"  # prefill-kernel route
    pipe = fa.HipAsymmetricProjectionPipeline(None)
    with pytest.raises(fa.FlatHipError) as e:
        pipe.encode_pre_rotated_k_decode_kv_reuse(None, None, None, None, None, None, None)
    assert e.value.variant == "CandidateNotEnabled"
    assert "external FLAT candidate M48 was not enabled" in str(e.value)
    assert fa.HipAsymmetricProjectionPipeline.with_decode_kv_reuse(None, True).decode_kv_reuse


def test_append_batched_validation():
    bt = np.array([[0, 1]], np.int32)
    st = np.array([20], np.int32)

    def call(bt=bt, st=st, app=8, pages=4, ps=16, D=64):
        return _variant(fa.lib().fa_paged_append_batched(
            None, bt.ctypes.data, bt.shape[1], st.ctypes.data, st.shape[0], app, ps, pages, 2, D,
            FAKE, FAKE, 1 << 30, FAKE, FAKE, 1 << 30, None, fa.DTYPE_BF16))
    assert call(app=20) == "CapacityExceeded"
    assert call(bt=np.array([[0, 7]], np.int32)) == "InvalidPage"
    assert call(D=60) == "UnsupportedHeadDim"
    assert call() == "NullArgument"


def _backward(shape=(2, 8, 2, 5, 16), dtype=fa.DTYPE_F32, fwd=None, grads=None, cfg=None):
    sh = L.GroupedShapeC(*shape)
    lay = L.BackwardLayoutC()
    rc = fa.lib().fa_backward_grouped_layout(ctypes.byref(sh), dtype, ctypes.byref(lay))
    if rc:
        return _variant(rc)
    fwd = lay.packed_forward_bytes if fwd is None else fwd
    grads = lay.gradient_bytes if grads is None else grads
    return _variant(fa.lib().fa_backward_grouped_recompute(
        None, FAKE, fwd, FAKE, grads, ctypes.byref(sh),
        ctypes.byref(cfg or L.ConfigC(0, 0, 0.0)), dtype))


def test_backward_layout_matches_reference_offsets():
    """GroupedBackwardRecomputeLayout src/wgpu_backward_grouped.rs:28-55 (element offsets,
    times 4 bytes for f32): Q | K | V | dO | O | LSE and dQ | dK | dV."""
    lay = fa.grouped_backward_layout(fa.GroupedAttentionShape(2, 8, 2, 5, 16), fa.DTYPE_F32)
    qe, ke, le = 2 * 8 * 5 * 16, 2 * 2 * 5 * 16, 2 * 8 * 5
    assert (lay.q_elements, lay.kv_elements, lay.lse_elements) == (qe, ke, le)
    assert [lay.q_offset, lay.k_offset, lay.v_offset, lay.d_out_offset, lay.output_offset,
            lay.lse_offset] == [4 * x for x in (0, qe, qe + ke, qe + 2 * ke, 2 * qe + 2 * ke,
                                                3 * qe + 2 * ke)]
    assert lay.packed_forward_bytes == 4 * (3 * qe + 2 * ke + le)
    assert [lay.dq_offset, lay.dk_offset, lay.dv_offset, lay.gradient_bytes] == \
        [0, 4 * qe, 4 * (qe + ke), 4 * (qe + 2 * ke)]
    l16 = fa.grouped_backward_layout(fa.GroupedAttentionShape(2, 8, 2, 5, 16), fa.DTYPE_BF16)
    assert l16.lse_offset == 2 * (3 * qe + 2 * ke) and l16.gradient_bytes == 2 * (qe + 2 * ke)


def test_backward_validation_variants():
    """prepare src/wgpu_backward_grouped.rs:231-246 order: shape, buffers (forward then
    gradients), scale; then head-dim support; a null context is reported last."""
    assert _backward(shape=(0, 8, 2, 5, 16)) == "ZeroDimension"
    assert _backward(shape=(2, 6, 4, 5, 16)) == "InvalidHeadGrouping"
    assert _backward(shape=(2**40, 2**20, 1, 2**20, 16)) == "ShapeOverflow"
    assert _backward(fwd=100) == "BufferTooSmall"
    assert _backward(grads=100) == "BufferTooSmall"
    assert _backward(cfg=L.ConfigC(0, 1, -1.0)) == "InvalidScale"
    assert _backward(shape=(1, 2, 1, 8, 256)) == "UnsupportedHeadDim"
    assert _backward(shape=(1, 2, 1, 8, 12), dtype=fa.DTYPE_BF16) == "UnsupportedHeadDim"
    assert _backward(shape=(1, 2, 1, 8, 6)) == "NullArgument"
    assert _backward() == "NullArgument"
    # tests/m22_prepared_validation.rs:143: overprovisioned buffers pass validation
    assert _backward(fwd=1 << 30, grads=1 << 30, cfg=L.ConfigC(1, 1, 0.25)) == "NullArgument"


def test_mha_backward_layout_and_validation():
    """WgpuBackwardRecomputePipeline::layout src/wgpu_backward.rs:162-185 (Q|K|V|dO|O|LSE with
    five equal tensors) and encode's validation order :207-214."""
    sh = L.AttentionShapeC(2, 3, 5, 8)
    lay = L.BackwardLayoutC()
    assert fa.lib().fa_backward_layout_mha(ctypes.byref(sh), fa.DTYPE_F32, ctypes.byref(lay)) == 0
    t = 2 * 3 * 5 * 8
    assert lay.packed_forward_bytes == 4 * (5 * t + 30) and lay.gradient_bytes == 12 * t
    assert (lay.k_offset, lay.lse_offset, lay.dv_offset) == (4 * t, 20 * t, 8 * t)

    def call(shape=(2, 3, 5, 8), fwd=None, grads=None):
        s_ = L.AttentionShapeC(*shape)
        return _variant(fa.lib().fa_backward_recompute_mha(
            None, FAKE, lay.packed_forward_bytes if fwd is None else fwd, FAKE,
            lay.gradient_bytes if grads is None else grads, ctypes.byref(s_),
            ctypes.byref(L.ConfigC(1, 0, 0.0)), fa.DTYPE_F32))
    assert call(shape=(2, 0, 5, 8)) == "ZeroDimension"
    assert call(fwd=64) == "BufferTooSmall"
    assert call(grads=64) == "BufferTooSmall"
    assert call() == "NullArgument"


def test_diagnostic_probes_validate_arguments():
    """The measurement aids live in their own library (libflat_diag.so): they reject a null
    output, an unknown dtype and an unsupported number of loads in flight before touching a
    device, and the attention library exports none of them."""
    from flat_attention_amd import diag
    lib = diag.lib()
    out = ctypes.c_double()
    assert lib.fad_mfma_ceiling(0, 2, 0, None) == 50  # NullArgument
    assert lib.fad_mfma_ceiling(0, 3, 0, ctypes.byref(out)) == 29  # UnsupportedDtype
    assert lib.fad_stream_read(0, 5, ctypes.byref(out)) == 20  # Unavailable
    assert lib.fad_stream_read(0, 8, None) == 50
    assert not hasattr(fa.lib(), "fa_diag_mfma_ceiling")


# --------------------------------------------------------------------------- contract fuzz
# tests/m39_host_api_fuzz.rs drives 4096 arbitrary shapes and configs (dimensions 0, 1, the
# integer maximum, half of it plus one, 128, 129 or 1..65; scales absent, 0, -1, NaN, +inf or
# in (0, 1]) through the host contract and requires that nothing panics. The same sweep goes
# through the C ABI here: with a null context every call must return a known error status (the
# context is only reported after the arguments are valid, so no call reaches the device), and
# the pure host layout / scale functions must return a known status too.


class _Fuzz:
    """xorshift64 stream with the reference's seed and value classes (restated)."""

    def __init__(self, seed):
        self.x = seed

    def next(self):
        x = self.x
        x ^= (x << 13) & 0xFFFFFFFFFFFFFFFF
        x ^= x >> 7
        x ^= (x << 17) & 0xFFFFFFFFFFFFFFFF
        self.x = x
        return x

    def dimension(self):
        m = self.next() & 15
        if m < 6:
            return (0, 1, 2**64 - 1, 2**63 + 1, 128, 129)[m]
        return self.next() % 65 + 1

    def scale(self):
        m = self.next() & 7
        if m < 5:
            return (None, 0.0, -1.0, float("nan"), float("inf"))[m]
        return ((self.next() % 10_000) + 1.0) / 10_000.0


def test_host_contract_fuzz_fails_closed():
    known = set(L.STATUS)
    st = _Fuzz(0x6D39F0221BADC0DE)
    lib = fa.lib()
    lay = L.BackwardLayoutC()
    scale_out = ctypes.c_float()
    for case in range(4096):
        b, hq, hkv, s, d, off = (st.dimension() for _ in range(6))
        cfg = fa.FlatAttentionConfig(st.next() & 1 == 0, st.scale())
        dtype = (fa.DTYPE_F32, fa.DTYPE_F16, fa.DTYPE_BF16, 7)[st.next() & 3]
        q_bytes, kv_bytes, out_bytes = (st.next() % (1 << 41) for _ in range(3))
        rc = _gqa(fa.GroupedAttentionShape(b, hq, hkv, s, d), cfg, None, dtype, q_bytes,
                  kv_bytes, out_bytes)
        assert rc in known and rc != 0, (case, rc)
        ash = fa.AsymmetricGroupedAttentionShape(b, hq, hkv, s, st.dimension(), d, off)
        rc = lib.fa_forward_projection_asymmetric(None, FAKE, q_bytes, FAKE, FAKE, kv_bytes, FAKE,
                                                  out_bytes, ctypes.byref(ash.c()),
                                                  ctypes.byref(cfg.c()), None, 0, dtype)
        assert rc in known and rc != 0, (case, rc)
        rot = fa.AsymmetricRotaryEmbeddingConfig(st.scale() or 1e4, st.dimension(), off)
        rc = lib.fa_forward_projection_asymmetric_decode_kv_reuse(
            None, FAKE, q_bytes, FAKE, FAKE, kv_bytes, FAKE, out_bytes, ctypes.byref(ash.c()),
            ctypes.byref(cfg.c()), ctypes.byref(rot.c()), dtype)
        assert rc in known and rc != 0, (case, rc)
        assert lib.fa_resolved_scale(ctypes.byref(cfg.c()), d, ctypes.byref(scale_out)) in known
        rc = lib.fa_backward_grouped_layout(ctypes.byref(fa.GroupedAttentionShape(
            b, hq, hkv, s, d).c()), dtype, ctypes.byref(lay))
        assert rc in known, (case, rc)


# --------------------------------------------------------------------------- device fingerprint
def _record(name, arch="gfx950", driver=70000, cus=256, clock=2400000, mem=288 << 30):
    buf = ctypes.create_string_buffer(512)
    fp = ctypes.c_uint64()
    assert fa.lib().fa_device_record(name.encode(), arch.encode(), driver, cus, clock, mem, buf,
                                     512, ctypes.byref(fp)) == 0
    return buf.value.decode(), fp.value


def _fnv1a64(data: bytes) -> int:
    h = 0xCBF29CE484222325
    for byte in data:
        h = ((h ^ byte) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def test_device_fingerprint_is_deterministic_driver_sensitive_and_escaped():
    """src/runtime_telemetry.rs:197-215 (the reference's unit tests of the record): the hash is
    deterministic and changes with the driver; delimiters inside a value are escaped while UTF-8
    is kept; the hash is FNV-1a-64 of the record's bytes (offset basis 0xcbf29ce484222325,
    prime 0x100000001b3; the empty input hashes to the basis)."""
    rec, fp = _record("AMD Instinct MI355X")
    assert _record("AMD Instinct MI355X") == (rec, fp)
    assert _record("AMD Instinct MI355X", driver=70001)[1] != fp
    assert rec == "name=AMD Instinct MI355X;arch=gfx950;driver=70000;cus=256;clock_khz=2400000;mem=309237645312"
    assert fp == _fnv1a64(rec.encode())
    assert _fnv1a64(b"") == 0xCBF29CE484222325
    assert _fnv1a64(b"a") == 0xAF63DC4C8601EC8C  # published FNV-1a-64 test vector
    rec2, _ = _record("GPU été;a=b%")
    assert "name=GPU été%3ba%3db%25;" in rec2


def test_passive_telemetry_validates_like_the_forward():
    """The snapshot (runtime_telemetry, tests/m29_runtime_telemetry.rs) checks the shape, RoPE,
    head_dim and dtype as the forward does; a null context is reported last."""
    lib = fa.lib()
    t = L.TelemetryC()
    cfg = ctypes.byref(fa.FlatAttentionConfig(True).c())

    def gqa(shape, rot=None, dtype=fa.DTYPE_BF16, out=True):
        return _variant(lib.fa_forward_gqa_rope_telemetry(
            None, ctypes.byref(fa.GroupedAttentionShape(*shape).c()), cfg,
            ctypes.byref(rot.c()) if rot else None, dtype, ctypes.byref(t) if out else None))

    assert gqa((1, 4, 2, 8, 64), out=False) == "NullArgument"
    assert gqa((1, 4, 0, 8, 64)) == "ZeroDimension"
    assert gqa((1, 6, 4, 8, 64)) == "InvalidHeadGrouping"
    assert gqa((1, 4, 2, 8, 63), fa.RotaryEmbeddingConfig(1e4, 0)) == "InvalidRotaryHeadDim"
    assert gqa((1, 4, 2, 8, 64), fa.RotaryEmbeddingConfig(0.0, 0)) == "InvalidRotaryTheta"
    assert gqa((1, 4, 2, 8, 60)) == "UnsupportedHeadDim"
    assert gqa((1, 4, 2, 8, 64), dtype=5) == "UnsupportedDtype"
    assert gqa((1, 4, 2, 8, 64)) == "NullArgument"
    assert _variant(lib.fa_forward_mha_telemetry(
        None, ctypes.byref(fa.AttentionShape(1, 2, 3, 129).c()), cfg, fa.DTYPE_F32,
        ctypes.byref(t))) == "UnsupportedHeadDim"


def test_graph_calls_need_a_context_and_a_capture():
    lib = fa.lib()
    h = ctypes.c_void_p()
    assert _variant(lib.fa_graph_capture_begin(None)) == "NullArgument"
    assert _variant(lib.fa_graph_capture_end(None, ctypes.byref(h))) == "NullArgument"
    assert _variant(lib.fa_graph_launch(None, None)) == "NullArgument"
    assert lib.fa_graph_destroy(None) == 0


def test_m39_overflow_position_and_length_fail_closed():
    """overflow_position_and_length_fail_closed tests/m39_host_api_fuzz.rs:108: batch or
    q_heads at usize::MAX and a query position at usize::MAX fail validation (asymmetric shape
    B1 Hq4 Hkv2 q2 kv3 D8); buffers one element short are BufferTooSmall."""
    lib = fa.lib()
    cfg = ctypes.byref(fa.FlatAttentionConfig(True).c())
    M = 2**64 - 1

    def asym(shape, q_bytes=1 << 30, kv_bytes=1 << 30):
        sh = fa.AsymmetricGroupedAttentionShape(*shape)
        return _variant(lib.fa_forward_projection_asymmetric(
            None, FAKE, q_bytes, FAKE, FAKE, kv_bytes, FAKE, 1 << 30, ctypes.byref(sh.c()), cfg,
            None, 0, fa.DTYPE_F32))

    valid = (1, 4, 2, 2, 3, 8, 0)
    for bad in ((M, 4, 2, 2, 3, 8, 0), (1, M, 1, 2, 3, 8, 0)):
        assert asym(bad) not in ("Ok", "NullArgument"), bad
    # offset + query_len wraps past 2^64: must still be PositionOverflow
    assert asym((1, 4, 2, 2, 3, 8, M)) == "PositionOverflow"
    assert asym((1, 4, 2, 2, 3, 8, M - 1)) == "PositionOverflow"
    assert asym(valid, q_bytes=4 * 2 * 8 * 4 - 4) == "BufferTooSmall"
    assert asym(valid, kv_bytes=2 * 3 * 8 * 4 - 4) == "BufferTooSmall"
    assert asym(valid) == "NullArgument"


def test_sizes_near_the_top_of_u64_fail_closed():
    """Element counts whose byte sizes would wrap past 2^64 (and sums of positions or lengths
    that would) are rejected before any buffer check could pass on a wrapped size: the
    fail-closed rule of tests/m39_host_api_fuzz.rs:108 applied to every size product."""
    lib = fa.lib()
    # 2^27 * 1 * 2^28 * 128 = 2^62 elements: 2^64 bytes in f32
    assert _variant(_gqa(fa.GroupedAttentionShape(2**27, 1, 1, 2**28, 128))) == "ShapeOverflow"
    sh = fa.AsymmetricGroupedAttentionShape(2**27, 1, 1, 1, 2**28, 128, 0)
    assert _variant(lib.fa_forward_projection_asymmetric(
        None, FAKE, 1 << 30, FAKE, FAKE, 1 << 30, FAKE, 1 << 30, ctypes.byref(sh.c()),
        ctypes.byref(fa.FlatAttentionConfig(False).c()), None, 0, fa.DTYPE_F32)) == "ShapeOverflow"
    # decode: heads whose Q / pool byte sizes wrap
    assert _decode_prepare([[0, 1, 2]], [40], hq=2**60, hkv=2**60) == "ShapeOverflow"
    assert _decode_prepare([[0, 1, 2]], [40], hq=2**59, hkv=2**58) == "ShapeOverflow"
    # append: a length that would wrap the end position, heads that wrap the row size
    bt = np.array([[0, 1]], np.int32)
    st = np.array([20], np.int32)

    def app(n=8, hkv=2, D=64):
        return _variant(lib.fa_paged_append_batched(
            None, bt.ctypes.data, bt.shape[1], st.ctypes.data, 1, n, 16, 4, hkv, D,
            FAKE, FAKE, 1 << 30, FAKE, FAKE, 1 << 30, None, fa.DTYPE_BF16))
    assert app(n=2**64 - 10) == "CapacityExceeded"
    assert app(n=2**64 - 1) == "CapacityExceeded"
    assert app(hkv=2**61) == "ShapeOverflow"
    assert app() == "NullArgument"


def test_prepared_and_pipeline_types_are_publicly_nameable():
    """prepared_grouped_forward_type_is_publicly_nameable
    tests/m44_prepared_grouped_public_api.rs:6: the prepared forward (and the other pipeline
    types a caller names in signatures) are exported at the package top level."""
    for name in ("PreparedGroupedForward", "PreparedGroupedBackwardRecompute", "HipGraph",
                 "HipRotaryGroupedAttention", "HipAsymmetricProjectionPipeline",
                 "HipProjectionRotaryGroupedPipeline", "HipResidentDecodePipeline",
                 "HipPagedDecodePipeline", "PagedDecodePlan", "PagedChunkedPrefillPlan"):
        assert isinstance(getattr(fa, name), type), name
