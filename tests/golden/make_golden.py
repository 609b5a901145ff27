"""Writes the golden fixtures under tests/golden/ (inputs + expected outputs).

  q4_0_ref.npz   Q4_0 blocks and the fp32 values produced by the reference's
                 own CPU dequantizer (src/quant.cpp:49-60, compiled where it
                 lies by `make -C oracle ref`); plus the reference's fp16->fp32
                 conversion of every binary16 bit pattern.
  kquants_ref.npz  Q4_K and Q8_0 blocks and the reference's own CPU
                 dequantization of them (src/quant.cpp:64-105).
  kernels.npz    seeded inputs and oracle outputs for each kernel at small
                 shapes (the oracle is pinned by tests/test_oracle_*.py); GPU
                 tests compare against these committed values.

Run from the repository root after `make -C oracle` (with the reference tree
present for the *_ref.npz files):  python tests/golden/make_golden.py [q4_0 kquants kernels]
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

import oracle  # noqa: E402
import testutil as tu  # noqa: E402

# binary16 scale values that exercise every class of d: zeros, one, negative,
# subnormal (smallest, largest), largest normal, infinities, NaN.
SPECIAL_D = [0x0000, 0x8000, 0x3C00, 0xBC00, 0x0001, 0x03FF, 0x0400, 0x7BFF, 0xFBFF,
             0x7C00, 0xFC00, 0x7E00, 0x2E66, 0x1400, 0x5BFF]


def q4_0_fixture():
    if not oracle.ref_available():
        raise SystemExit("oracle/_ref/libjinf_ref.so missing: run `make -C oracle ref` first")
    r = tu.rng(40)
    d_bits, qs = [], []
    # every byte value 0..255 under every special scale
    for d in SPECIAL_D:
        for start in range(0, 256, 16):
            d_bits.append(d)
            qs.append(np.arange(start, start + 16, dtype=np.uint8))
    # random blocks: d = fp16(|N(0, 0.02)|), random nibbles
    n_rand = 256
    d_rand = np.abs(r.normal(0, 0.02, n_rand)).astype(np.float16).view(np.uint16)
    d_bits.extend(d_rand.tolist())
    qs.extend(r.integers(0, 256, size=(n_rand, 16), dtype=np.uint8))
    blocks = tu.q4_0_blocks(np.array(d_bits, np.uint16), np.array(qs, np.uint8))
    out = oracle.ref_dequant_q4_0(blocks)
    all_h = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    f16_ref = oracle.ref_f16_to_f32(all_h)
    np.savez_compressed(os.path.join(HERE, "q4_0_ref.npz"), blocks=blocks, out=out,
                        f16_bits=all_h.view(np.uint16), f16_to_f32=f16_ref)
    print("q4_0_ref.npz:", blocks.size // 18, "blocks")


def kquants_fixture():
    """Q4_K and Q8_0 blocks and the reference's own CPU dequantization of them
    (src/quant.cpp:64-105 via oracle/_ref)."""
    if not oracle.ref_available():
        raise SystemExit("oracle/_ref/libjinf_ref.so missing: run `make -C oracle ref` first")
    r = tu.rng(41)
    fx = {}
    for qtype, key in ((oracle.Q4_K, "q4_K"), (oracle.Q8_0, "q8_0")):
        e, nbytes = oracle.qtype_geometry(qtype)
        rand = tu.quant_table(r, qtype, 1, e * 96, 0.05).reshape(-1, nbytes)
        special = np.repeat(rand[:len(SPECIAL_D)], 1, axis=0).copy()
        special[:, 0:2] = np.array(SPECIAL_D, np.uint16).view(np.uint8).reshape(-1, 2)
        if qtype == oracle.Q4_K:  # dmin through the same special values, reversed
            special[:, 2:4] = np.array(SPECIAL_D[::-1], np.uint16).view(np.uint8).reshape(-1, 2)
        blocks = np.concatenate([rand, special]).reshape(-1)
        fx[key + "_blocks"] = blocks
        fx[key + "_out"] = oracle.ref_dequant(qtype, blocks)
    np.savez_compressed(os.path.join(HERE, "kquants_ref.npz"), **fx)
    print("kquants_ref.npz:", {k: v.shape for k, v in fx.items()})


def kernels_fixture():
    fx = {}
    # config 1: RMSNorm fp32, 1 x 4096, eps 1e-5, x ~ N(0,1), gamma ~ N(1,0.05) f32
    r = tu.rng(1)
    x = tu.normal(r, (1, 4096), 0.0, 1.0, np.float32)
    w = tu.normal(r, (4096,), 1.0, 0.05, np.float32)
    fx["rms1_x"], fx["rms1_w"] = x, w
    fx["rms1_y"] = oracle.rmsnorm_rows(x, w, 1e-5)
    # fused residual + RMSNorm fp16 [8, 512], fp16 gamma
    r = tu.rng(3)
    res = tu.normal(r, (8, 512))
    dx = tu.normal(r, (8, 512))
    g = tu.normal(r, (512,), 1.0, 0.05)
    fx["frn_res"], fx["frn_x"], fx["frn_w"] = res, dx, g
    fx["frn_res_out"], fx["frn_y"] = oracle.residual_rmsnorm_rows(res, dx, g, 1e-5)
    # RoPE fp16: q [16, 4*128], k [16, 2*128], positions up to 8191, theta 500000
    r = tu.rng(2)
    q = tu.normal(r, (16, 4 * 128))
    k = tu.normal(r, (16, 2 * 128))
    pos = r.integers(0, 8192, size=16).astype(np.int32)
    fx["rope_q"], fx["rope_k"], fx["rope_pos"] = q, k, pos
    fx["rope_q_out"], fx["rope_k_out"] = oracle.rope_rows(q, k, 128, pos, 0, 500000.0)
    # SwiGLU fp16 [8, 1024], gate/up ~ N(0, 2)
    r = tu.rng(4)
    gate = tu.normal(r, (8, 1024), 0.0, 2.0)
    up = tu.normal(r, (8, 1024), 0.0, 2.0)
    fx["sw_gate"], fx["sw_up"] = gate, up
    fx["sw_out"] = oracle.swiglu(gate, up)
    # masked softmax fp32 [3 seqs x 4 heads, 1024], logits ~ N(0, 3), len = pos + 1
    r = tu.rng(5)
    s = tu.normal(r, (12, 1024), 0.0, 3.0, np.float32)
    lens = np.array([1, 517, 1024], np.int32)
    fx["sm_x"], fx["sm_lens"] = s, lens
    fx["sm_y"] = oracle.softmax_rows(s, lens, 4, 1.0, out=np.full_like(s, np.nan))
    # Q4_0 gather -> fp16: table 64 x 256, 32 ids (one out of range)
    r = tu.rng(6)
    table = tu.q4_0_table(r, 64, 256)
    ids = r.integers(0, 64, size=32).astype(np.int32)
    ids[7] = 64
    fx["emb_table"], fx["emb_ids"] = table, ids
    fx["emb_out"] = oracle.embed_q4_0(table, ids, 256, np.float16)
    np.savez_compressed(os.path.join(HERE, "kernels.npz"), **fx)
    print("kernels.npz:", sorted(fx))


if __name__ == "__main__":
    # optional arguments pick fixtures by name (q4_0, kquants, kernels); default all
    makers = {"q4_0": q4_0_fixture, "kquants": kquants_fixture, "kernels": kernels_fixture}
    for name in sys.argv[1:] or list(makers):
        makers[name]()
