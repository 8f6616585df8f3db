"""Writes the small golden fixtures under tests/golden/ from the CPU oracle.

The reference crate holds no stored golden vectors (every reference test compares against its
in-process Rust oracle), so these fixtures are produced by this repo's C restatement of that
oracle after it is pinned by tests/test_oracle.py (float64 two-pass softmax, closed forms,
RoPE identities). tests/test_golden.py re-derives every fixture and checks it against float64.
Run: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
import oracle  # noqa: E402


def main():
    out = {}
    # MHA B1 H2 N128 D64 causal f32, inputs N(0,1) from seeds 1,2,3
    B, H, S, D = 1, 2, 128, 64
    q, k, v = (oracle.fill_normal(B * H * S * D, s) for s in (1, 2, 3))
    o, l = oracle.forward(q, k, v, B, H, S, D, True)
    np.savez(os.path.join(HERE, "cfg1_mha_causal.npz"), q=q, k=k, v=v, o=o, lse=l,
             shape=np.array([B, H, S, D]))
    # GQA + fused RoPE, B1 Hq4 Hkv2 N48 D32, theta 1e4, offset 5, causal
    B, hq, hkv, S, D = 1, 4, 2, 48, 32
    q = oracle.fill_normal(B * hq * S * D, 4)
    k, v = oracle.fill_normal(B * hkv * S * D, 5), oracle.fill_normal(B * hkv * S * D, 6)
    o, l = oracle.forward_grouped_rope(q, k, v, B, hq, hkv, S, D, True, 1e4, 5)
    np.savez(os.path.join(HERE, "gqa_rope_small.npz"), q=q, k=k, v=v, o=o, lse=l,
             shape=np.array([B, hq, hkv, S, D]), theta=np.float32(1e4), offset=5)
    # paged decode: 3 sequences, page 4, shuffled pool of 9 pages, Hq4 Hkv2 D16
    rng = np.random.default_rng(7)
    ps, hq, hkv, D = 4, 4, 2, 16
    lens = np.array([5, 12, 1], np.int32)
    perm = rng.permutation(9).astype(np.int32)
    bt = np.array([[perm[0], perm[1], 0], [perm[2], perm[3], perm[4]], [perm[5], 0, 0]], np.int32)
    kp = oracle.fill_normal(9 * ps * hkv * D, 8)
    vp = oracle.fill_normal(9 * ps * hkv * D, 9)
    qd = oracle.fill_normal(3 * hq * D, 10)
    o, l = oracle.paged_decode(qd, kp, vp, 9, ps, bt, lens, hq, hkv, D, True, 1e4)
    np.savez(os.path.join(HERE, "paged_decode_small.npz"), q=qd, k_pool=kp, v_pool=vp,
             block_tables=bt, ctx_lens=lens, o=o, lse=l, dims=np.array([ps, hq, hkv, D, 9]))
    # chunked prefill (projection layout), B2 Hq4 Hkv1 S20 D16, chunk 6, offset 3
    B, hq, hkv, S, D = 2, 4, 1, 20, 16
    q = oracle.fill_normal(B * S * hq * D, 11)
    k, v = oracle.fill_normal(B * S * hkv * D, 12), oracle.fill_normal(B * S * hkv * D, 13)
    o, l = oracle.chunked_prefill(q, k, v, B, hq, hkv, S, D, True, 1e4, 3, 6)
    np.savez(os.path.join(HERE, "chunked_small.npz"), q=q, k=k, v=v, o=o, lse=l,
             shape=np.array([B, hq, hkv, S, D]), chunk=6, offset=3)


if __name__ == "__main__":
    main()
