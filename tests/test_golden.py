"""Golden fixtures (tests/golden/, written by make_golden.py from the pinned oracle): the
oracle reproduces them bit-for-bit, each is independently within float64 tolerance, and the
GPU path matches them (gpu tests)."""
import os

import numpy as np
import pytest

import oracle
from conftest import assert_close
from test_oracle import naive64, rope64

import flat_attention_amd as fa

G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(G, name), allow_pickle=False)


def test_cfg1_fixture():
    f = load("cfg1_mha_causal.npz")
    B, H, S, D = f["shape"].tolist()
    o, l = oracle.forward(f["q"], f["k"], f["v"], B, H, S, D, True)
    assert np.array_equal(o, f["o"]) and np.array_equal(l, f["lse"])
    eo, el = naive64(f["q"], f["k"], f["v"], B, H, H, S, D, True)
    assert_close("O", f["o"], eo, 2e-6, 2e-6)
    assert_close("LSE", f["lse"], el, 2e-6, 2e-6)


def test_gqa_rope_fixture():
    f = load("gqa_rope_small.npz")
    B, hq, hkv, S, D = f["shape"].tolist()
    th, off = float(f["theta"]), int(f["offset"])
    o, l = oracle.forward_grouped_rope(f["q"], f["k"], f["v"], B, hq, hkv, S, D, True, th, off)
    assert np.array_equal(o, f["o"]) and np.array_equal(l, f["lse"])
    qr = rope64(f["q"], B * hq * S, 1, D, th, off + np.tile(np.arange(S), B * hq)).astype(np.float32)
    kr = rope64(f["k"], B * hkv * S, 1, D, th, off + np.tile(np.arange(S), B * hkv)).astype(np.float32)
    eo, el = naive64(qr, kr, f["v"], B, hq, hkv, S, D, True)
    assert_close("O", f["o"], eo, 1e-5, 1e-5)
    assert_close("LSE", f["lse"], el, 1e-5, 1e-5)


def test_paged_decode_fixture():
    f = load("paged_decode_small.npz")
    ps, hq, hkv, D, pages = f["dims"].tolist()
    o, l = oracle.paged_decode(f["q"], f["k_pool"], f["v_pool"], pages, ps, f["block_tables"],
                               f["ctx_lens"], hq, hkv, D, True, 1e4)
    assert np.array_equal(o, f["o"]) and np.array_equal(l, f["lse"])
    width = hkv * D
    for s, n in enumerate(f["ctx_lens"].tolist()):
        rows = [f["block_tables"][s, t // ps] * ps + t % ps for t in range(n)]
        kc = np.concatenate([f["k_pool"][r * width:(r + 1) * width] for r in rows])
        vc = np.concatenate([f["v_pool"][r * width:(r + 1) * width] for r in rows])
        qr = rope64(f["q"][s * hq * D:(s + 1) * hq * D], 1, hq, D, 1e4, [n - 1]).astype(np.float32)
        eo, el = naive64(qr, kc, vc, 1, hq, hkv, n, D, True, qpos_off=n - 1, kv_len=n,
                         layout="proj", q_len=1)
        assert_close("O", f["o"][s * hq * D:(s + 1) * hq * D], eo, 1e-5, 1e-5)
        assert_close("LSE", f["lse"][s * hq:(s + 1) * hq], el, 1e-5, 1e-5)


def test_chunked_fixture():
    f = load("chunked_small.npz")
    B, hq, hkv, S, D = f["shape"].tolist()
    o, l = oracle.chunked_prefill(f["q"], f["k"], f["v"], B, hq, hkv, S, D, True, 1e4,
                                  int(f["offset"]), int(f["chunk"]))
    assert np.array_equal(o, f["o"]) and np.array_equal(l, f["lse"])


# ------------------------------------------------------------------------------ GPU

@pytest.mark.gpu
def test_gpu_matches_golden_fixtures(hip):
    f = load("cfg1_mha_causal.npz")
    B, H, S, D = f["shape"].tolist()
    r = fa.HipFlatAttention(hip, fa.DTYPE_F32).forward(f["q"], f["k"], f["v"],
                                                       fa.AttentionShape(B, H, S, D),
                                                       fa.FlatAttentionConfig(True))
    assert_close("cfg1 O", r.output, f["o"], 2e-5, 1e-4)
    assert_close("cfg1 LSE", r.lse, f["lse"], 2e-5, 1e-4)

    f = load("gqa_rope_small.npz")
    B, hq, hkv, S, D = f["shape"].tolist()
    r = fa.HipRotaryGroupedAttention(hip, fa.DTYPE_F32).forward(
        f["q"], f["k"], f["v"], fa.GroupedAttentionShape(B, hq, hkv, S, D),
        fa.FlatAttentionConfig(True), fa.RotaryEmbeddingConfig(float(f["theta"]), int(f["offset"])))
    assert_close("gqa O", r.output, f["o"], 2e-5, 1e-4)
    assert_close("gqa LSE", r.lse, f["lse"], 2e-5, 1e-4)

    f = load("paged_decode_small.npz")
    ps, hq, hkv, D, pages = f["dims"].tolist()
    plan = fa.PagedDecodePlan(hip, f["block_tables"], f["ctx_lens"], ps, pages, hq, hkv, D,
                              fa.FlatAttentionConfig(True), 1e4, fa.DTYPE_F32)
    bufs = [fa.DeviceBuffer.from_array(hip, f[n]) for n in ("q", "k_pool", "v_pool")]
    out = fa.DeviceBuffer(hip, plan.layout().combined_bytes)
    plan.launch(*bufs, out)
    r = fa.download_attention(out, plan.layout(), fa.DTYPE_F32)
    assert_close("decode O", r.output, f["o"], 2e-5, 1e-4)
    assert_close("decode LSE", r.lse, f["lse"], 2e-5, 1e-4)

    f = load("chunked_small.npz")
    B, hq, hkv, S, D = f["shape"].tolist()
    shape = fa.GroupedAttentionShape(B, hq, hkv, S, D)
    pipe = fa.HipChunkedProjectionPrefillPipeline(hip, fa.DTYPE_F32)
    out = pipe.create_output_buffer(shape)
    pipe.encode(*(fa.DeviceBuffer.from_array(hip, f[n]) for n in ("q", "k", "v")), out, shape,
                fa.FlatAttentionConfig(True), fa.RotaryEmbeddingConfig(1e4, int(f["offset"])),
                int(f["chunk"]))
    r = fa.download_attention(out, pipe.layout(shape), fa.DTYPE_F32)
    assert_close("chunked O", r.output, f["o"], 2e-5, 1e-4)
    assert_close("chunked LSE", r.lse, f["lse"], 2e-5, 1e-4)
