"""Benchmark: achieved HBM bandwidth of jinf's per-layer elementwise / reduction
kernels on one MI355X, with the CPU oracle timed beside it.

A step is one pass of the hot path over one batch of synthetic input.  The
default workload, llama3-8b-layer, is every Llama-3-8B-shaped configuration of
the path:
    rope     Q [512, 32, 128] + K [512, 8, 128] fp16, positions 0..511, theta 5e5
    norm     fused residual add + RMSNorm fp16 [2048, 4096], eps 1e-5
    swiglu   silu(gate) * up fp16 [2048, 14336]
    gather   Q4_0 token-embedding gather 4096 ids of 128256 x 4096 -> fp16
and the same run also times config 5, the Llama-3-70B decode chain for 64
sequences (residual+RMSNorm, RoPE 64/8 heads, masked fp32 softmax over
len = pos + 1, SwiGLU, residual add), reported under "config5".
`--workload llama3-70b-decode` runs config 5 alone.

value = algorithmic bytes of a step / GPU time of a step (GB/s).  Algorithmic
bytes count every input read once and every output written once.  Inputs are
resident in HBM before timing; each kernel rotates over enough buffer sets
(>= 512 MiB of distinct memory per kernel) that no launch can be served from
the 256 MB Infinity Cache.  Times come from HIP events on the stream the
kernels run on: the K steps are captured as one HIP graph and the replay is
bracketed by two events (ms_per_step); each kernel's average launch duration
is timed the same way over max(K, --kernel-launches) back-to-back launches of
that kernel alone in one graph (kernels.*.us, roofline.avg_launch_us), so the
graph's own start-up cost is spread over as many launches as a decode loop
would run.

Ceilings: every kernel is timed beside a bandwidth probe (include/jinf/
probe_hip.h) that moves the same bytes in the same launch geometry with no
arithmetic; kernels.*.frac_of_ceiling = probe time / kernel time.

Prints ONE JSON line (rank 0).  `--gpus N` with N > 1 exits: this build runs
on one GPU.
"""
import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "jetson-inference_amd"))

PEAK_GBS = 8000.0
ROTATE_BYTES = 512 << 20
METRIC = "achieved HBM GB/s & % of 8 TB/s peak per kernel; rows/sec at Llama-8B shape"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# --------------------------------------------------------------------------
# workloads: each kernel is (name, bytes per launch, rows per launch,
# row unit, list of per-set launch closures)
# --------------------------------------------------------------------------

class Kernel:
    """One kernel of a step: its launch closures over rotating buffer sets,
    algorithmic bytes and rows per launch, the bandwidth probe of each set
    (the same bytes in the same geometry, no arithmetic), and (for the CPU
    baseline) the tensors of set 0 with the oracle call that computes the
    same thing."""

    def __init__(self, name, nbytes, rows, row_unit, launches, hip_name, set0=(), cpu=None,
                 probes=None, probe_name=None):
        self.name, self.nbytes, self.rows, self.row_unit = name, nbytes, rows, row_unit
        self.launches, self.hip_name = launches, hip_name
        self.set0, self.cpu = set0, cpu
        self.probes, self.probe_name = probes, probe_name
        # probe variants tried for the ceiling: (units per lane, cross-lane exchange)
        self.probe_upls = ((1, True), (2, True), (4, True), (1, False), (2, False), (4, False))
        self.key = name              # unique name across the run (CPU baseline)
        self.i = 0
        self.ms = 0.0
        self.n = 0
        self.ceil_ms = None
        self.ceil_upl = None

    def run(self, probe=0):
        """One launch over the next buffer set: the kernel, or (probe = a
        (units per lane, exchange) variant) its bandwidth probe."""
        if probe:
            self.probes[self.i % len(self.probes)](probe)
        else:
            self.launches[self.i % len(self.launches)]()
        self.i += 1


def n_sets(footprint_bytes):
    """Buffer sets whose distinct memory together covers ROTATE_BYTES."""
    return max(2, -(-ROTATE_BYTES // footprint_bytes))


def randn16(torch, shape, mu, sigma, g):
    return (torch.randn(shape, generator=g, device="cuda", dtype=torch.float32) * sigma
            + mu).to(torch.float16)


def q4_0_table(torch, n_vocab, n_embd, g):
    nb = n_embd // 32
    t = torch.randint(0, 256, (n_vocab, nb, 18), generator=g, device="cuda",
                      dtype=torch.int32).to(torch.uint8)
    d = (torch.randn((n_vocab, nb), generator=g, device="cuda") * 0.02).abs().to(torch.float16)
    t[:, :, 0:2] = d.view(torch.uint8).view(n_vocab, nb, 2)
    return t.view(n_vocab, nb * 18)


def build_rope(torch, jinf, g, T, nh, nkv, hd, positions, keep):
    nbytes = T * (nh + nkv) * hd * 2 * 2 + T * 4
    sets, probes = [], []
    for _ in range(n_sets(T * (nh + nkv) * hd * 2)):
        q = randn16(torch, (T, nh * hd), 0.0, 1.0, g)
        k = randn16(torch, (T, nkv * hd), 0.0, 1.0, g)
        p = positions.clone()
        keep.append((q, k, p))
        sets.append(lambda q=q, k=k, p=p: jinf.rope_rows(q, k, hd, p, 0, 500000.0))
        probes.append(lambda u, q=q, k=k: jinf.ops.probe_rows_inplace(q, k, *u))
    return Kernel("rope", nbytes, T, "token rows", sets, "rope_vec_kernel", keep[-len(sets)],
                  lambda o, q, k, p: o.rope_rows(q, k, hd, p, 0, 500000.0),
                  probes, "probe_rows_inplace_kernel")


def build_norm(torch, jinf, g, T, H, keep):
    nbytes = 4 * T * H * 2 + H * 2
    sets, probes = [], []
    for _ in range(n_sets(3 * T * H * 2)):
        r = randn16(torch, (T, H), 0.0, 1.0, g)
        x = randn16(torch, (T, H), 0.0, 1.0, g)
        w = randn16(torch, (H,), 1.0, 0.05, g)
        y = torch.empty_like(x)
        keep.append((r, x, w, y))
        sets.append(lambda r=r, x=x, w=w, y=y: jinf.residual_rmsnorm_rows(r, x, w, 1e-5, out=y))
        probes.append(lambda u, r=r, x=x, y=y: jinf.ops.probe_stream(r, r, y, x, *u))
    return Kernel("residual_rmsnorm", nbytes, T, "token rows", sets, "rmsnorm_vec_kernel",
                  keep[-len(sets)][:3], lambda o, r, x, w: o.residual_rmsnorm_rows(r, x, w, 1e-5),
                  probes, "probe_stream_kernel")


def build_swiglu(torch, jinf, g, T, F, keep):
    nbytes = 3 * T * F * 2
    sets, probes = [], []
    for _ in range(n_sets(nbytes)):
        gt = randn16(torch, (T, F), 0.0, 2.0, g)
        up = randn16(torch, (T, F), 0.0, 2.0, g)
        o = torch.empty_like(gt)
        keep.append((gt, up, o))
        sets.append(lambda gt=gt, up=up, o=o: jinf.swiglu(gt, up, out=o))
        probes.append(lambda u, gt=gt, up=up, o=o: jinf.ops.probe_stream(o, gt, None, up, *u))
    return Kernel("swiglu", nbytes, T, "token rows", sets, "ew_vec_kernel",
                  keep[-len(sets)][:2], lambda o, gt, up: o.swiglu(gt, up),
                  probes, "probe_stream_kernel")


def build_residual_add(torch, jinf, g, T, H, keep):
    nbytes = 3 * T * H * 2
    sets, probes = [], []
    for _ in range(n_sets(2 * T * H * 2)):
        a = randn16(torch, (T, H), 0.0, 1.0, g)
        b = randn16(torch, (T, H), 0.0, 1.0, g)
        keep.append((a, b))
        sets.append(lambda a=a, b=b: jinf.residual_add(a, b))
        probes.append(lambda u, a=a, b=b: jinf.ops.probe_stream(a, a, None, b, *u))
    return Kernel("residual_add", nbytes, T, "token rows", sets, "ew_vec_kernel",
                  keep[-len(sets)], lambda o, a, b: o.residual_add(a, b),
                  probes, "probe_stream_kernel")


def build_gather(torch, jinf, g, n_vocab, n_embd, n_ids, keep):
    row_bytes = n_embd // 32 * 18
    nbytes = n_ids * row_bytes + n_ids * 4 + n_ids * n_embd * 2
    # one table, as config 4 has (a second table doubles the address range
    # the random rows spread over, and its translation misses cost the
    # gather about 7%: 8.0-8.1 against 7.5-7.7 us); each set draws its own
    # uniform ids, and the output rows rotate over >= 512 MiB
    table = q4_0_table(torch, n_vocab, n_embd, g)
    tables = [table]
    keep.append(tables)
    sets, probes = [], []
    for i in range(n_sets(n_ids * n_embd * 2)):
        ids = torch.randint(0, n_vocab, (n_ids,), generator=g, device="cuda", dtype=torch.int32)
        o = torch.empty((n_ids, n_embd), dtype=torch.float16, device="cuda")
        t = table
        keep.append((ids, o))
        sets.append(lambda t=t, ids=ids, o=o: jinf.embed_q4_0(t, ids, n_embd, torch.float16, out=o))
        probes.append(lambda u, t=t, ids=ids, o=o: jinf.ops.probe_gather(o, t, ids, row_bytes, *u))
    import numpy as np
    return Kernel("q4_0_gather", nbytes, n_ids, "token ids", sets, "embed_q4_0_kernel",
                  (tables[0], keep[-len(sets)][0]),
                  lambda o, t, ids: o.embed_q4_0(t, ids, n_embd, np.float16),
                  probes, "probe_gather_kernel")


def build_softmax(torch, jinf, g, n_seq, n_heads, max_len, keep):
    pos = torch.randint(0, max_len, (n_seq,), generator=g, device="cuda", dtype=torch.int32)
    lens = pos + 1
    live = int(lens.sum().item())
    nbytes = 8 * n_heads * live + n_seq * 4
    # sets are counted by the bytes a launch touches (the live prefixes), not
    # by the padded rows: only touched lines can be left in the 256 MB cache
    sets, probes = [], []
    for _ in range(n_sets(nbytes)):
        s = torch.randn((n_seq * n_heads, max_len), generator=g, device="cuda") * 3.0
        o = torch.empty_like(s)
        lc = lens.clone()
        keep.append((s, o, lc))
        sets.append(lambda s=s, o=o, lc=lc: jinf.softmax_rows(s, lc, n_heads, 1.0, out=o))
        probes.append(lambda u, s=s, o=o, lc=lc: jinf.ops.probe_rows_ragged(o, s, lc, n_heads))
    k = Kernel("masked_softmax", nbytes, n_seq * n_heads, "score rows", sets,
               "softmax_vec_kernel", (keep[-len(sets)][0], lens),
               lambda o, s, lc: o.softmax_rows(s, lc, n_heads, 1.0),
               probes, "probe_rows_ragged_kernel")
    k.probe_upls = ((4, True),)  # the softmax's own 4 units per lane
    return k


def build_attention(torch, jinf, g, name, n_seq, max_ctx, nh, nkv, hd, lens, kv_dtype, keep):
    """GQA decode attention over an n_seq-sequence KV cache.  Algorithmic bytes:
    every live K and V row of every kv head read once, q read, out written."""
    es = 2 if kv_dtype == torch.float16 else 4
    live = int(lens.sum().item())
    nbytes = 2 * live * nkv * hd * es + 2 * n_seq * nh * hd * 4 + n_seq * 4
    n_past = int(lens[0].item())  # the drop-in takes the length on the host
    sets = []
    for _ in range(n_sets(nbytes)):  # counted by touched bytes (live K/V rows)
        k = torch.randn((n_seq, max_ctx, nkv * hd), generator=g, device="cuda").to(kv_dtype)
        v = torch.randn((n_seq, max_ctx, nkv * hd), generator=g, device="cuda").to(kv_dtype)
        q = torch.randn((n_seq, nh * hd), generator=g, device="cuda") * 2.0
        o = torch.empty((n_seq, nh * hd), dtype=torch.float32, device="cuda")
        lc = lens.clone()
        ws = jinf.attention_workspace(n_seq, nh, hd, max_ctx)
        keep.append((q, k, v, lc, o, ws))
        if n_seq == 1 and kv_dtype == torch.float32:  # the reference's drop-in
            sets.append(lambda q=q, k=k, v=v, o=o: jinf.cuda_attention(
                o, q, k, v, hd, nh, nkv, n_past, max_ctx))
        else:
            sets.append(lambda q=q, k=k, v=v, lc=lc, o=o, ws=ws: jinf.attention_decode(
                q, k, v, lc, nh, nkv, out=o, workspace=ws))
    return Kernel(name, nbytes, n_seq, "sequences", sets,
                  "attn_mfma_kernel" if kv_dtype == torch.float16 else "attn_decode_kernel",
                  keep[-len(sets)][:4],
                  lambda o, q, k, v, lc: o.attention(q, k, v, lc, nh, nkv, hd))


# GGUF block geometry (values, bytes) and where each format keeps its binary16
# scales (byte offsets within the block).
QGEOM = {2: (32, 18, (0,)), 8: (32, 34, (0,)), 12: (256, 144, (0, 2)), 14: (256, 210, (208,))}


def quant_table(torch, qtype, rows, cols, g):
    """Random weight rows of a GGUF block type: every byte uniform, then the
    binary16 scales set to fp16(|N(0, 0.02)|)."""
    if qtype == 2:
        return q4_0_table(torch, rows, cols, g)
    elems, nbytes, scale_offs = QGEOM[qtype]
    nb = cols // elems
    t = torch.randint(0, 256, (rows, nb, nbytes), generator=g, device="cuda",
                      dtype=torch.int32).to(torch.uint8)
    for off in scale_offs:
        d = (torch.randn((rows, nb), generator=g, device="cuda") * 0.02).abs().to(torch.float16)
        t[:, :, off:off + 2] = d.view(torch.uint8).view(rows, nb, 2)
    return t.view(rows, nb * nbytes)


def build_matvec(torch, jinf, g, name, rows, cols, keep, qtype=2):
    """Dequant-GEMV y = W x at batch 1 (fp32 x, y), W in qtype blocks."""
    elems, nbytes_blk, _ = QGEOM[qtype]
    nbytes = rows * (cols // elems) * nbytes_blk + cols * 4 + rows * 4
    sets = []
    for _ in range(n_sets(nbytes)):
        W = quant_table(torch, qtype, rows, cols, g)
        x = torch.randn(cols, generator=g, device="cuda")
        y = torch.empty(rows, dtype=torch.float32, device="cuda")
        keep.append((W, x, y))
        sets.append(lambda W=W, x=x, y=y: jinf.matvec(W, x, qtype, y))
    return Kernel(name, nbytes, rows, "output rows", sets, f"matvec_kernel<{qtype}",
                  keep[-len(sets)][:2], lambda o, W, x: o.matvec(qtype, W, x))


# --------------------------------------------------------------------------
# geometry-free attainable rate: the fastest of many launch layouts of a plain
# stream with a kernel's read:write mix, at the kernel's own size
# --------------------------------------------------------------------------

# mix -> (inputs, outputs, first output written in place of the first input)
FLAT_MIXES = {"2:1": (2, 1, False), "2:1 in place": (2, 1, True),
              "2:2 in place": (2, 2, True), "1:1 in place": (1, 1, True), "1:1": (1, 1, False)}
KERNEL_MIX = {"rope": "1:1 in place", "residual_rmsnorm": "2:2 in place", "swiglu": "2:1",
              "residual_add": "2:1 in place", "masked_softmax": "1:1", "q4_0_gather": "gather",
              "gemv_q": "read", "gemv_k": "read", "gemv_v": "read", "gemv_o": "read",
              "gemv_gate": "read", "gemv_up": "read", "gemv_down": "read"}
# (units per lane, store order, lanes per workgroup, workgroups: 0 = one pass
# over the data, else a grid-stride loop over that many).  Store order: False,
# every store after the lane's loads; True, after a cross-lane exchange; 2 (two
# outputs), the first output straight after its own loads and the second after
# the exchange, as a row norm stores r' before its reduction and y after it.
FLAT_LAYOUTS = tuple((u, x, b, gr) for u in (1, 2, 4) for x in (True, False, 2)
                     for b, gr in ((64, 0), (128, 0), (256, 0), (512, 0), (1024, 0),
                                   (256, 2048), (1024, 512)))
GATHER_LAYOUTS = ((1, True), (2, True), (4, True), (1, False), (2, False), (4, False))
GATHER_VOCAB = 128256  # rows of the table the gather mix reads from
READ_LAYOUTS = tuple(lay for lay in FLAT_LAYOUTS if not lay[1])  # no stores to exchange for


def build_flat(torch, jinf, mix, nbytes, keep):
    """Buffer sets of a plain stream of about `nbytes` algorithmic bytes with
    read:write mix `mix` (rotated over >= 512 MiB of touched memory); its
    probe variants are the launch layouts FLAT_LAYOUTS.  "gather" is the Q4_0
    gather's row mix (2304-byte rows read : 8192-byte rows written)."""
    if mix == "gather":
        # n rows of a vocabulary-sized table (config 4's 128256 rows, 295 MB),
        # in a random order, each into the next output row; the rotated sets
        # read disjoint rows, so no launch finds another's rows in the cache
        ri, ro = 2304, 8192
        n = max(1, nbytes // (ri + ro + 4))
        ns = n_sets(n * (ri + ro))
        rows = max(ns * n, GATHER_VOCAB)
        t = torch.ones((rows, ri), dtype=torch.uint8, device="cuda")
        perm = torch.randperm(rows, device="cuda").to(torch.int32)
        keep.append((t, perm))
        probes = []
        for s in range(ns):
            o = torch.empty((n, ro), dtype=torch.uint8, device="cuda")
            ids = perm[s * n:(s + 1) * n].contiguous()
            keep.append((o, ids))
            probes.append(lambda u, t=t, o=o, ids=ids:
                          jinf.ops.probe_gather(o, t, ids, ri, *u))
        k = Kernel("row gather", n * (ri + ro + 4), 0, "", [], "probe_gather_kernel",
                   probes=probes, probe_name="probe_gather_kernel")
        k.probe_upls = GATHER_LAYOUTS
        return k
    if mix == "read":
        # a GEMV's weight traffic: reads only
        n_units = max(1, nbytes // 16)
        sink = torch.zeros(4, dtype=torch.int32, device="cuda")
        probes = []
        for _ in range(n_sets(16 * n_units)):
            t = torch.ones(n_units * 4, dtype=torch.float32, device="cuda")
            keep.append((t, sink))
            probes.append(lambda lay, t=t: jinf.ops.probe_read_layout(t, sink, lay[0], lay[2],
                                                                      lay[3]))
        k = Kernel("flat read", 16 * n_units, 0, "", [], "probe_read_kernel", probes=probes,
                   probe_name="probe_read_kernel")
        k.probe_upls = READ_LAYOUTS
        return k
    ni, no, inplace = FLAT_MIXES[mix]
    n_units = max(1, nbytes // (16 * (ni + no)))
    touched = 16 * n_units * (ni + no - (1 if inplace else 0))
    probes = []
    for _ in range(n_sets(touched)):
        ins = [torch.ones(n_units * 4, dtype=torch.float32, device="cuda") for _ in range(ni)]
        outs = [torch.empty(n_units * 4, dtype=torch.float32, device="cuda")
                for _ in range(no - (1 if inplace else 0))]
        if inplace:
            outs.insert(0, ins[0])
        keep.append((ins, outs))
        probes.append(lambda lay, o0=outs[0], i0=ins[0], o1=outs[1] if no > 1 else None,
                      i1=ins[1] if ni > 1 else None:
                      jinf.ops.probe_stream_layout(o0, i0, o1, i1, *lay))
    k = Kernel(f"flat {mix}", 16 * n_units * (ni + no), 0, "", [], "probe_flat_kernel",
               probes=probes, probe_name="probe_flat_kernel")
    k.probe_upls = FLAT_LAYOUTS
    return k


def attainable(torch, jinf, timed, mix, nbytes, n_launch):
    """(us per launch scaled to nbytes, layout) of the fastest layout of a
    plain stream with read:write mix `mix` moving about nbytes."""
    scratch = []
    fk = build_flat(torch, jinf, mix, nbytes, scratch)
    torch.cuda.synchronize()
    best = None
    for lay in fk.probe_upls:
        ms = timed(n_launch, [fk], probe=lay)
        if best is None or ms < best[0]:
            best = (ms, lay)
    us = best[0] / n_launch * 1e3 * nbytes / fk.nbytes
    del fk, scratch
    torch.cuda.empty_cache()
    return us, best[1]


CURVE_MB = (2.0, 2.36, 3.15, 4.0, 4.21, 8.0, 10.49, 11.01, 16.0, 32.0, 43.01, 64.0, 67.12,
            128.0, 136.49, 176.16, 256.0, 512.0)


def stream_curve(torch, jinf, timed, n_launch):
    """Text table: best attainable stream rate per read:write mix and size."""
    lines = ["attainable HBM stream rate on one MI355X: the fastest of "
             f"{len(FLAT_LAYOUTS)} launch layouts (flat mixes), {len(GATHER_LAYOUTS)} "
             f"(row gather) or {len(READ_LAYOUTS)} (read only) per point, each timed over "
             f"{n_launch} back-to-back launches in one HIP graph, buffer sets rotated over "
             ">= 512 MiB of touched memory",
             "layout = (units per lane, store order: False after the loads, True after a "
             "cross-lane exchange, 2 first output after its own loads[, lanes per workgroup, "
             "workgroups (0 = one pass, else grid-stride)])", ""]
    for mix in list(FLAT_MIXES) + ["gather", "read"]:
        lines.append(f"mix {mix}:")
        lines.append(f"  {'MB':>8} {'us':>9} {'GB/s':>8} {'% of 8 TB/s':>12}  layout")
        for mb in CURVE_MB:
            nb = int(mb * 1e6)
            us, lay = attainable(torch, jinf, timed, mix, nb, n_launch)
            gbs = nb / (us * 1e-6) / 1e9
            lines.append(f"  {mb:8.2f} {us:9.3f} {gbs:8.1f} {100 * gbs / PEAK_GBS:11.1f}%  "
                         f"{lay}")
            log(f"curve {mix} {mb} MB: {us:.3f} us")
        lines.append("")
    return "\n".join(lines)


def config5(torch, jinf, g, keep):
    """the Llama-3-70B decode chain for 64 sequences."""
    pos = torch.randint(0, 8192, (64,), generator=g, device="cuda", dtype=torch.int32)
    ks = [build_norm(torch, jinf, g, 64, 8192, keep),
          build_rope(torch, jinf, g, 64, 64, 8, 128, pos, keep),
          build_softmax(torch, jinf, g, 64, 64, 8192, keep),
          build_swiglu(torch, jinf, g, 64, 28672, keep),
          build_residual_add(torch, jinf, g, 64, 8192, keep)]
    for k in ks:
        k.key = "config5_" + k.name
    cfg = {"workload": "llama3-70b-decode", "shapes": "Llama-3-70B decode, 64 sequences: hidden "
           "8192, 64/8 heads x 128, FFN 28672, score rows 4096 x stride 8192, len = pos + 1, "
           "pos ~ U[0, 8192)", "storage": "f16 activations, f32 scores", "baseline_configs": [5]}
    return ks, cfg


def workload(name, torch, jinf, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    keep = []
    if name == "llama3-8b-layer":
        ks = [build_rope(torch, jinf, g, 512, 32, 8, 128,
                         torch.arange(512, dtype=torch.int32, device="cuda"), keep),
              build_norm(torch, jinf, g, 2048, 4096, keep),
              build_swiglu(torch, jinf, g, 2048, 14336, keep),
              build_gather(torch, jinf, g, 128256, 4096, 4096, keep)]
        cfg = {"workload": name, "shapes": "Llama-3-8B: hidden 4096, 32/8 heads x 128, FFN 14336, "
               "vocab 128256; RoPE T=512, norm/SwiGLU T=2048, 4096 token ids",
               "storage": "f16 activations, Q4_0 table", "baseline_configs": [2, 3, 4]}
    elif name == "llama3-70b-decode":
        ks, cfg = config5(torch, jinf, g, keep)
    elif name == "calibrate":
        # the bandwidth probes of configs 2-5 alone (for a rocprof summary)
        k8, _ = config5(torch, jinf, g, keep)
        ks = [build_rope(torch, jinf, g, 512, 32, 8, 128,
                         torch.arange(512, dtype=torch.int32, device="cuda"), keep),
              build_norm(torch, jinf, g, 2048, 4096, keep),
              build_swiglu(torch, jinf, g, 2048, 14336, keep),
              build_gather(torch, jinf, g, 128256, 4096, 4096, keep)] + k8
        for k in ks:  # every probe variant, one after the other
            k.launches = [lambda f=f, u=u: f(u) for u in k.probe_upls for f in k.probes]
            k.hip_name = k.probe_name
        cfg = {"workload": name, "shapes": "the bandwidth probes of BASELINE configs 2-5",
               "baseline_configs": [2, 3, 4, 5]}
    elif name == "llama3-8b-gemv":
        H, F, KV = 4096, 14336, 1024
        ks = [build_matvec(torch, jinf, g, "gemv_q", H, H, keep),
              build_matvec(torch, jinf, g, "gemv_k", KV, H, keep),
              build_matvec(torch, jinf, g, "gemv_v", KV, H, keep),
              build_matvec(torch, jinf, g, "gemv_o", H, H, keep),
              build_matvec(torch, jinf, g, "gemv_gate", F, H, keep),
              build_matvec(torch, jinf, g, "gemv_up", F, H, keep),
              build_matvec(torch, jinf, g, "gemv_down", H, F, keep)]
        cfg = {"workload": name, "dtype": "f32 math, Q4_0 weights (fp16 scales), f32 x and y",
               "shapes": "Llama-3-8B layer projections at batch 1 (decode): "
               "q/o 4096x4096, k/v 1024x4096, gate/up 14336x4096, down 4096x14336, Q4_0 "
               "weights, fp32 x/y", "storage": "Q4_0 weights, f32 vectors",
               "baseline_configs": [], "note": "batch-1 dequant-GEMVs, beside the hot path"}
    elif name in ("llama3-8b-gemv-q4_k_m", "llama3-8b-gemv-q8_0"):
        H, F, KV = 4096, 14336, 1024
        if name.endswith("q8_0"):
            qt = dict.fromkeys(("q", "k", "v", "o", "gate", "up", "down"), 8)
            desc = "Q8_0 weights"
        else:  # Q4_K_M: Q4_K, with Q6_K for attn_v and ffn_down
            qt = dict(q=12, k=12, v=14, o=12, gate=12, up=12, down=14)
            desc = "Q4_K weights, Q6_K for v and down (Q4_K_M)"
        shapes = dict(q=(H, H), k=(KV, H), v=(KV, H), o=(H, H), gate=(F, H), up=(F, H),
                      down=(H, F))
        ks = [build_matvec(torch, jinf, g, "gemv_" + p, rows, cols, keep, qt[p])
              for p, (rows, cols) in shapes.items()]
        cfg = {"workload": name, "dtype": f"f32 math, {desc} (fp16 scales), f32 x and y",
               "shapes": "Llama-3-8B layer projections at batch 1 (decode): "
               "q/o 4096x4096, k/v 1024x4096, gate/up 14336x4096, down 4096x14336, " + desc,
               "storage": desc + ", f32 vectors", "baseline_configs": [],
               "note": "batch-1 dequant-GEMVs, beside the hot path"}
    elif name == "llama3-70b-attention":
        pos = torch.randint(0, 8192, (64,), generator=g, device="cuda", dtype=torch.int32)
        ks = [build_attention(torch, jinf, g, "gqa_attention", 64, 8192, 64, 8, 128, pos + 1,
                              torch.float16, keep)]
        cfg = {"workload": name, "dtype": "f32 math, f16 KV cache, f32 q and out",
               "shapes": "Llama-3-70B decode attention, 64 sequences: 64/8 heads x 128, "
               "KV cache [64, 8192, 8 x 128] fp16, len = pos + 1, pos ~ U[0, 8192)",
               "storage": "f16 KV cache", "baseline_configs": [5],
               "note": "decode attention at config 5's sequences and lengths"}
    elif name == "llama3-8b-attention-b1":
        lens = torch.full((1,), 4096, dtype=torch.int32, device="cuda")
        ks = [build_attention(torch, jinf, g, "gqa_attention_b1", 1, 4096, 32, 8, 128, lens,
                              torch.float32, keep)]
        cfg = {"workload": name, "dtype": "f32",
               "shapes": "Llama-3-8B decode attention through the reference's drop-in "
               "jinf_cuda_attention: one sequence, 32/8 heads x 128, fp32 cache, n_past 4096",
               "storage": "f32 KV cache", "baseline_configs": [],
               "note": "decode attention, batch 1, the reference's drop-in"}
    elif name == "llama3-8b-attention-b1-f16":
        lens = torch.full((1,), 8192, dtype=torch.int32, device="cuda")
        ks = [build_attention(torch, jinf, g, "gqa_attention_b1_f16", 1, 8192, 32, 8, 128, lens,
                              torch.float16, keep)]
        cfg = {"workload": name, "dtype": "f32 math, f16 KV cache, f32 q and out",
               "shapes": "Llama-3-8B decode attention at batch 1 through jinf_attention_decode "
               "with a workspace (context split over 1024-position chunks): 32/8 heads x 128, "
               "fp16 cache, 8192 positions",
               "storage": "f16 KV cache", "baseline_configs": [],
               "note": "decode attention, batch 1, split contexts"}
    elif name in ("rope", "norm", "swiglu", "gather", "softmax"):
        b = {"rope": lambda: build_rope(torch, jinf, g, 512, 32, 8, 128,
                                        torch.arange(512, dtype=torch.int32, device="cuda"), keep),
             "norm": lambda: build_norm(torch, jinf, g, 2048, 4096, keep),
             "swiglu": lambda: build_swiglu(torch, jinf, g, 2048, 14336, keep),
             "gather": lambda: build_gather(torch, jinf, g, 128256, 4096, 4096, keep),
             "softmax": lambda: build_softmax(torch, jinf, g, 64, 64, 8192, keep)}[name]
        ks = [b()]
        cfg = {"workload": name, "shapes": "single kernel, BASELINE.json shape"}
    else:
        raise SystemExit(f"unknown workload {name}")
    return ks, cfg, keep


# --------------------------------------------------------------------------
# decode engine: Llama-3-8B-shaped random weights resident in HBM, one token
# per step through jinf_hip_engine (include/jinf/engine_hip.h)
# --------------------------------------------------------------------------

ENGINE_MODELS = {
    # llama.cpp's Q4_0 file layout: Q4_0 everywhere, Q6_K output
    "llama3-8b-decode": dict(mat=dict.fromkeys(("attn_q", "attn_k", "attn_v", "attn_output",
                                                "ffn_gate", "ffn_up", "ffn_down"), 2),
                             embd=2, out=14, desc="Q4_0 weights, Q6_K output"),
    # Q4_K_M: Q4_K, with Q6_K for attn_v and ffn_down, Q6_K output
    "llama3-8b-decode-q4_k_m": dict(mat=dict(attn_q=12, attn_k=12, attn_v=14, attn_output=12,
                                             ffn_gate=12, ffn_up=12, ffn_down=14),
                                    embd=12, out=14,
                                    desc="Q4_K weights, Q6_K for attn_v, ffn_down and output"),
    # the same Q4_0 model decoding 32 sequences at once (jinf_hip_batch_*)
    "llama3-8b-decode-batch": dict(mat=dict.fromkeys(("attn_q", "attn_k", "attn_v",
                                                      "attn_output", "ffn_gate", "ffn_up",
                                                      "ffn_down"), 2),
                                   embd=2, out=14, batch=32,
                                   desc="Q4_0 weights, Q6_K output"),
    # the Q4_K_M model decoding 32 sequences at once
    "llama3-8b-decode-batch-q4_k_m": dict(mat=dict(attn_q=12, attn_k=12, attn_v=14,
                                                   attn_output=12, ffn_gate=12, ffn_up=12,
                                                   ffn_down=14),
                                          embd=12, out=14, batch=32,
                                          desc="Q4_K weights, Q6_K for attn_v, ffn_down and "
                                               "output"),
}
LLAMA3_8B = dict(n_layers=32, n_embd=4096, n_heads=32, n_heads_kv=8, n_ff=14336,
                 n_vocab=128256, rope_freq_base=500000.0, rms_norm_eps=1e-5)
PROMPT = [1, 450, 4696, 310, 2834, 338]   # the reference bench's prompt ids


def engine_weights(torch, g, spec, hp):
    """{GGUF name: (device tensor, qtype)} of a random Llama-3-8B-shaped model."""
    H, F, V = hp["n_embd"], hp["n_ff"], hp["n_vocab"]
    KV = hp["n_heads_kv"] * (H // hp["n_heads"])
    shapes = dict(attn_q=(H, H), attn_k=(KV, H), attn_v=(KV, H), attn_output=(H, H),
                  ffn_gate=(F, H), ffn_up=(F, H), ffn_down=(H, F))
    W = {"token_embd.weight": (quant_table(torch, spec["embd"], V, H, g), spec["embd"]),
         "output.weight": (quant_table(torch, spec["out"], V, H, g), spec["out"]),
         "output_norm.weight": (torch.randn(H, generator=g, device="cuda") * 0.05 + 1.0, 0)}
    for L in range(hp["n_layers"]):
        for n in ("attn_norm", "ffn_norm"):
            W[f"blk.{L}.{n}.weight"] = (torch.randn(H, generator=g, device="cuda") * 0.05 + 1.0, 0)
        for n, (rows, cols) in shapes.items():
            W[f"blk.{L}.{n}.weight"] = (quant_table(torch, spec["mat"][n], rows, cols, g),
                                        spec["mat"][n])
    return W


def engine_cpu_baseline(W, hp, spec, threads, budget_s):
    """The oracle's decode loop (oracle/engine.py) on a host copy of the
    weights: the prompt, then greedy tokens until the budget is spent."""
    sys.path.insert(0, ROOT)
    import oracle
    from oracle import engine as oeng

    oracle.set_threads(threads)
    Wh = {k: (t.cpu().numpy(), qt) for k, (t, qt) in W.items()}
    dec = oeng.Decoder(hp, Wh, max_context=64, kv_type=1)
    times = []
    tok = PROMPT[0]
    t_end = time.perf_counter() + budget_s
    for i in range(60):
        t0 = time.perf_counter()
        lg = dec.step(tok)
        times.append(time.perf_counter() - t0)
        tok = PROMPT[i + 1] if i + 1 < len(PROMPT) else oeng.first_argmax(lg)
        if time.perf_counter() > t_end and len(times) >= 2:
            break
    med = sorted(times)[len(times) // 2]
    return med, len(times)


def batch_bench(args, torch, jinf_amd, spec):
    """n_seq sequences decoded together: prompt through forward, then
    `steps` greedy steps through jinf_hip_batch_generate (tokens fed back on
    the device, one synchronization at the end)."""
    hp = dict(LLAMA3_8B)
    n_seq = args.batch or spec["batch"]
    max_ctx = 1024
    g = torch.Generator(device="cuda")
    g.manual_seed(args.seed)
    W = engine_weights(torch, g, spec, hp)
    torch.cuda.synchronize()
    from jinf_amd.engine import Batch, Engine

    e = Engine(hp, W, 16, jinf_amd.F16)
    b = Batch(e, n_seq, max_ctx, jinf_amd.F16)
    b.use_graph(not args.no_graph)
    wbytes = e.step_weight_bytes - weight_row_bytes(spec["embd"], hp["n_embd"])
    wbytes += n_seq * weight_row_bytes(spec["embd"], hp["n_embd"])  # one embedding row each
    kvd = hp["n_heads_kv"] * hp["n_embd"] // hp["n_heads"]
    log(f"batch of {n_seq} ready: {wbytes / 1e9:.3f} GB of weights read per step")
    t0 = time.perf_counter()
    for tok in PROMPT:
        b.forward([tok] * n_seq)
    prefill_s = time.perf_counter() - t0
    b.generate(max(1, args.warmup))
    start_pos = b.n_past(0)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    out = b.generate(args.steps)
    dec_s = time.perf_counter() - t0
    emitted = int((out >= 0).sum())
    ms_step = dec_s / args.steps * 1e3
    mean_ctx = start_pos + (args.steps + 1) / 2
    kv_bytes = n_seq * 2 * hp["n_layers"] * kvd * 2 * mean_ctx  # fp16 K and V rows read
    step_bytes = wbytes + kv_bytes
    gbs = step_bytes / (ms_step * 1e-3) / 1e9
    tok_s = emitted / dec_s
    log(f"{args.steps} steps x {n_seq} sequences: {ms_step:.3f} ms per step, "
        f"{tok_s:.0f} tokens/s")
    # prompt processing: one sequence's 512-token prompt through
    # jinf_hip_batch_prefill (chunks of n_seq tokens per step), after one
    # untimed run
    import ctypes
    import numpy as np
    n_pf = min(args.prompt_tokens, max_ctx)
    ids = np.ascontiguousarray(
        np.random.default_rng(args.seed).integers(0, hp["n_vocab"], n_pf).astype(np.int32))
    lptr = ctypes.c_void_p()
    pf_s = None
    for _ in range(2 if n_pf > 0 else 0):
        b.reset(0)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        rc = jinf_amd.lib().jinf_hip_batch_prefill(b._h, 0, ids.ctypes.data, n_pf,
                                                  ctypes.byref(lptr))
        pf_s = time.perf_counter() - t0
        if rc != 0:
            raise SystemExit(f"jinf_hip_batch_prefill failed ({rc})")
    if n_pf > 0:
        log(f"prefill of {n_pf} tokens in chunks of {n_seq}: {pf_s * 1e3:.2f} ms, "
            f"{n_pf / pf_s:.0f} tokens/s")
    b.close()
    e.close()
    cpu = None
    if args.cpu_seconds > 0:
        threads = args.cpu_threads or min(16, os.cpu_count() or 1)
        try:
            med, runs = engine_cpu_baseline(W, hp, spec, threads, args.cpu_seconds)
            cpu = {"value": round(1.0 / med, 4), "unit": "tokens/s", "cores": threads,
                   "kind": "port", "runs": runs,
                   "sample": f"oracle decode loop (oracle/engine.py, C kernels -O3, {threads} "
                             f"OpenMP threads), one sequence on a host copy of the same weights: "
                             f"median of {runs} tokens, {args.cpu_seconds:.0f} s budget (the "
                             f"reference decodes one sequence at a time)",
                   "cpu_model": cpu_model()}
        except Exception as exc:  # the baseline is reported, never required
            log(f"cpu baseline failed: {exc!r}")
    out_line = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32 math (fp16 x fp16 products on the matrix cores), " + spec["desc"] +
                 ", f16 KV cache",
        "data": "synthetic: random Llama-3-8B-shaped weights (seeded torch RNG on device), "
                "the reference prompt for every sequence, then greedy tokens",
        "config": {"workload": args.workload,
                   "shapes": "Llama-3-8B: 32 layers, hidden 4096, 32/8 heads x 128, FFN 14336, "
                             f"vocab 128256, {n_seq} sequences decoded together",
                   "storage": spec["desc"] + f", f16 KV cache (max_context {max_ctx} per sequence)",
                   "step": "one token for every sequence through every layer, captured HIP "
                           "graph replayed per step (jinf_hip_batch_generate)",
                   "tokens_per_s": round(tok_s, 1),
                   "prefill_6_steps_ms": round(prefill_s * 1e3, 3),
                   "prompt_tokens": n_pf,
                   "prompt_ms": round(pf_s * 1e3, 3) if n_pf else None,
                   "prompt_tokens_per_s": round(n_pf / pf_s, 1) if n_pf else None,
                   "weight_bytes_per_step": wbytes,
                   "kv_bytes_per_step_mean": int(kv_bytes),
                   "context": [start_pos, start_pos + args.steps],
                   "note": "the engine's batched decode loop, batched KV cache"},
        "frac_of_peak": round(gbs / PEAK_GBS, 4),
        "launch": "eager stream" if args.no_graph else "HIP graph per step",
        "wall_s_timed": round(dec_s, 4),
        "roofline": {"bound": "hbm", "kernel": "decode step (every kernel of one batched step)",
                     "achieved": round(gbs, 1), "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_GBS, 4), "bytes_per_launch": int(step_bytes),
                     "avg_launch_us": round(ms_step * 1e3, 3),
                     "traffic": traffic_from_profiles("decode_step", args.workload)},
        "cpu_baseline": cpu,
    }
    if args.calibrate_copy:
        calibrate_copy(torch)
    print(json.dumps(out_line), flush=True)


def f4_figures(args, torch, jinf_amd):
    """The engine rows (f1 GEMVs, f2 attention, f4 loop) on the Q4_0
    Llama-3-8B-shaped model of `--workload llama3-8b-decode`, measured inside
    the default run: batch-1 decode (K tokens in one forward call, one
    captured graph per token) and the 32-sequence batched decode (K steps of
    jinf_hip_batch_generate).  Weight GB/s = weight bytes read per step / step
    time; the KV-cache rows read are reported beside it."""
    from jinf_amd.engine import Batch, Engine

    spec = ENGINE_MODELS["llama3-8b-decode"]
    hp = dict(LLAMA3_8B)
    g = torch.Generator(device="cuda")
    g.manual_seed(args.seed)
    W = engine_weights(torch, g, spec, hp)
    torch.cuda.synchronize()
    kvd = hp["n_heads_kv"] * hp["n_embd"] // hp["n_heads"]
    erow = weight_row_bytes(spec["embd"], hp["n_embd"])
    steps = max(8, min(args.steps, 32))
    out = {"model": "Llama-3-8B-shaped, 32 layers, " + spec["desc"] + ", f16 KV cache, random "
                    "weights (--workload llama3-8b-decode / llama3-8b-decode-batch)",
           "steps_timed": steps}
    with Engine(hp, W, 1024, jinf_amd.F16) as e:
        e.use_graph(not args.no_graph)
        wbytes = e.step_weight_bytes
        e.forward(PROMPT)
        e.forward([PROMPT[-1]] * 2)
        toks = [int(t) for t in torch.randint(0, hp["n_vocab"], (steps,), generator=g,
                                              device="cuda").cpu()]
        start = e.n_past
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e.forward(toks)
        ms = (time.perf_counter() - t0) / steps * 1e3
        kv = 2 * hp["n_layers"] * kvd * 2 * (start + (steps + 1) / 2)
        out["batch1"] = {"ms_per_token": round(ms, 4), "tokens_per_s": round(1e3 / ms, 1),
                         "weight_bytes": wbytes, "kv_bytes_mean": int(kv),
                         "weight_GB/s": round(wbytes / (ms * 1e-3) / 1e9, 1),
                         "frac_of_8TBs": round((wbytes + kv) / (ms * 1e-3) / 1e9 / PEAK_GBS, 4),
                         "context": [start, start + steps]}
        n_seq = 32
        with Batch(e, n_seq, 256, jinf_amd.F16) as b:
            b.use_graph(not args.no_graph)
            for tok in PROMPT:
                b.forward([tok] * n_seq)
            b.generate(2)
            start = b.n_past(0)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            b.generate(steps)
            ms = (time.perf_counter() - t0) / steps * 1e3
            wb = wbytes - erow + n_seq * erow
            kv = n_seq * 2 * hp["n_layers"] * kvd * 2 * (start + (steps + 1) / 2)
            out["batch32"] = {"ms_per_step": round(ms, 4),
                              "tokens_per_s": round(n_seq * 1e3 / ms, 1),
                              "weight_bytes": wb, "kv_bytes_mean": int(kv),
                              "weight_GB/s": round(wb / (ms * 1e-3) / 1e9, 1),
                              "frac_of_8TBs": round((wb + kv) / (ms * 1e-3) / 1e9 / PEAK_GBS, 4),
                              "context": [start, start + steps]}
    del W
    torch.cuda.empty_cache()
    return out


def weight_row_bytes(qtype, n):
    elems, nbytes = {2: (32, 18), 8: (32, 34), 12: (256, 144), 14: (256, 210)}[qtype]
    return n // elems * nbytes


def engine_bench(args, torch, jinf_amd):
    spec = ENGINE_MODELS[args.workload]
    if "batch" in spec:
        return batch_bench(args, torch, jinf_amd, spec)
    hp = dict(LLAMA3_8B)
    max_ctx = 8192
    g = torch.Generator(device="cuda")
    g.manual_seed(args.seed)
    W = engine_weights(torch, g, spec, hp)
    torch.cuda.synchronize()
    from jinf_amd.engine import Engine

    e = Engine(hp, W, max_ctx, jinf_amd.F16)
    e.use_graph(not args.no_graph)
    wbytes = e.step_weight_bytes
    kvd = hp["n_heads_kv"] * hp["n_embd"] // hp["n_heads"]
    log(f"engine ready: {wbytes / 1e9:.3f} GB of weights read per token")

    # prefill as in the reference bench (6 prompt tokens, one forward call)
    t0 = time.perf_counter()
    e.forward(PROMPT)
    prefill_s = time.perf_counter() - t0
    for _ in range(max(1, args.warmup)):
        e.forward([PROMPT[-1]])
    # timed decode steps: K tokens in one forward call (each step is the
    # captured graph; one synchronization at the end)
    toks = [int(t) for t in torch.randint(0, hp["n_vocab"], (args.steps,), generator=g,
                                          device="cuda").cpu()]
    start_pos = e.n_past
    t0 = time.perf_counter()
    e.forward(toks)
    dec_s = time.perf_counter() - t0
    ms_tok = dec_s / args.steps * 1e3
    mean_ctx = start_pos + (args.steps + 1) / 2
    kv_bytes = 2 * hp["n_layers"] * kvd * 2 * mean_ctx      # fp16 K and V rows read
    step_bytes = wbytes + kv_bytes
    # greedy generation through jinf_hip_engine_generate (per-token host
    # read of the argmax, as the reference's generate loop)
    n_gen = min(args.steps, max_ctx - e.n_past - 1)
    t0 = time.perf_counter()
    out = e.generate([], n_gen)
    gen_s = time.perf_counter() - t0
    log(f"token steps decoded in this run: {e.n_past}")
    # a 512-token prompt: batched prefill (steps of 64 tokens on the batched
    # GEMVs) against the token-by-token forward call, each from position 0
    n_pf = min(args.prompt_tokens, max_ctx)
    pf_toks = [int(t) for t in torch.randint(0, hp["n_vocab"], (max(n_pf, 1),), generator=g,
                                             device="cuda").cpu()]
    pf_ms = {"prefill": float("nan"), "forward": float("nan")}
    for how in ("prefill", "forward", "prefill") if n_pf > 0 else ():
        # the first prefill is untimed warm-up
        e.reset()
        t0 = time.perf_counter()
        getattr(e, how)(pf_toks)
        pf_ms[how] = (time.perf_counter() - t0) * 1e3
    if n_pf > 0:
        log(f"{n_pf}-token prompt: prefill {pf_ms['prefill']:.1f} ms, "
            f"forward {pf_ms['forward']:.1f} ms")
    e.close()

    gbs = step_bytes / (ms_tok * 1e-3) / 1e9
    cpu = None
    if args.cpu_seconds > 0:
        threads = args.cpu_threads or min(16, os.cpu_count() or 1)
        try:
            med, runs = engine_cpu_baseline(W, hp, spec, threads, args.cpu_seconds)
            cpu = {"value": round(wbytes / med / 1e9, 3), "unit": "GB/s", "cores": threads,
                   "kind": "port", "tokens_per_s": round(1.0 / med, 4), "runs": runs,
                   "sample": f"oracle decode loop (oracle/engine.py, C kernels -O3, {threads} "
                             f"OpenMP threads) on a host copy of the same weights: the prompt "
                             f"and greedy tokens, median of {runs} tokens, "
                             f"{args.cpu_seconds:.0f} s budget",
                   "cpu_model": cpu_model()}
        except Exception as exc:  # the baseline is reported, never required
            log(f"cpu baseline failed: {exc!r}")
    out_line = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_tok, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32 math, " + spec["desc"] + ", f16 KV cache",
        "data": "synthetic: random Llama-3-8B-shaped weights (seeded torch RNG on device, block "
                "bytes uniform, fp16 scales |N(0,0.02)|), random token ids",
        "config": {"workload": args.workload,
                   "shapes": "Llama-3-8B: 32 layers, hidden 4096, 32/8 heads x 128, FFN 14336, "
                             "vocab 128256, batch 1 decode",
                   "storage": spec["desc"] + ", f16 KV cache (max_context 8192)",
                   "step": "one token through every layer (jinf_hip_engine_forward), captured "
                           "HIP graph replayed per token",
                   "tokens_per_s": round(1e3 / ms_tok, 2),
                   "generate_tokens_per_s": round(len(out) / gen_s, 2) if out else None,
                   "generated": len(out),
                   "prefill_6_tokens_ms": round(prefill_s * 1e3, 3),
                   "prompt_tokens": n_pf,
                   "prompt_prefill_ms": round(pf_ms["prefill"], 3) if n_pf else None,
                   "prompt_forward_ms": round(pf_ms["forward"], 3) if n_pf else None,
                   "prompt_prefill_tokens_per_s":
                       round(n_pf / pf_ms["prefill"] * 1e3, 1) if n_pf else None,
                   "weight_bytes_per_token": wbytes,
                   "kv_bytes_per_token_mean": int(kv_bytes),
                   "context": [start_pos, start_pos + args.steps],
                   "baseline_configs": [], "note": "the engine forward loop"},
        "frac_of_peak": round(gbs / PEAK_GBS, 4),
        "launch": "eager stream" if args.no_graph else "HIP graph per token",
        "wall_s_timed": round(dec_s, 4),
        "roofline": {"bound": "hbm", "kernel": "decode step (every kernel of one token)",
                     "achieved": round(gbs, 1), "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_GBS, 4), "bytes_per_launch": int(step_bytes),
                     "avg_launch_us": round(ms_tok * 1e3, 3),
                     "traffic": traffic_from_profiles("decode_step", args.workload)},
        "cpu_baseline": cpu,
    }
    if args.calibrate_copy:
        calibrate_copy(torch)
    print(json.dumps(out_line), flush=True)


# --------------------------------------------------------------------------
# CPU baseline: the oracle (a C restatement of the reference arithmetic) on
# the host cores, same workload shapes, on a copy of buffer set 0
# --------------------------------------------------------------------------

def cpu_baseline(ks, threads, budget_s):
    """Median seconds per run of every kernel's oracle call at `threads`
    threads, on host copies of buffer set 0, within about budget_s."""
    sys.path.insert(0, ROOT)
    import oracle

    oracle.set_threads(threads)
    out = {}
    for k in ks:
        arrays = [t.cpu().numpy() for t in k.set0]
        fn = lambda: k.cpu(oracle, *arrays)  # noqa: E731
        fn()  # warm-up
        times = []
        t_end = time.perf_counter() + budget_s / len(ks)
        while True:
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
            if time.perf_counter() > t_end and len(times) >= 10:
                break
        out[k.key] = (sorted(times)[len(times) // 2], len(times))
    oracle.set_threads(1)
    return out


def host_threads(args):
    """(threads of the all-cores run, cores this process may use)."""
    try:
        aff = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        aff = os.cpu_count() or 1
    return (args.cpu_threads or min(16, aff)), aff


def oracle_build():
    """The -march of the oracle library this host loads."""
    sys.path.insert(0, ROOT)
    import oracle

    return "-march=x86-64-v4" if oracle.ORACLE_PATH.endswith("_v4.so") else "-march=x86-64-v3"


def cpu_baseline_both(ks, ks70, args):
    """The oracle timed at 1 thread (the reference's CPU code is
    single-threaded) and at every core this run may use (at most 16, the GPU
    box's share for one GPU), for the step's kernels and config 5's."""
    n_all, aff = host_threads(args)
    budget = args.cpu_seconds / 2
    runs = {1: cpu_baseline(ks + ks70, 1, budget), n_all: cpu_baseline(ks + ks70, n_all, budget)}

    def rate(kl, t):
        sec = sum(runs[t][k.key][0] for k in kl)
        return round(sum(k.nbytes for k in kl) / sec / 1e9, 3), round(sec, 5)

    def per(t):
        return {k.key: round(k.nbytes / runs[t][k.key][0] / 1e9, 3) for k in ks + ks70}

    def per_us(t):
        return {k.key: round(runs[t][k.key][0] * 1e6, 1) for k in ks + ks70}

    def per_rows(t):
        return {k.key: round(k.rows / runs[t][k.key][0], 1) for k in ks + ks70}

    v_all, s_all = rate(ks, n_all)
    v_one, s_one = rate(ks, 1)
    out = {"value": v_all, "unit": "GB/s", "cores": n_all, "kind": "port",
           "s_per_step": s_all, "per_kernel_GBs": per(n_all), "per_kernel_us": per_us(n_all),
           "per_kernel_rows_per_s": per_rows(n_all),
           "single_thread": {"value": v_one, "unit": "GB/s", "cores": 1, "s_per_step": s_one,
                             "per_kernel_GBs": per(1), "per_kernel_us": per_us(1),
                             "per_kernel_rows_per_s": per_rows(1)},
           "runs": {k.key: [runs[1][k.key][1], runs[n_all][k.key][1]] for k in ks + ks70},
           "host_cores": os.cpu_count(), "usable_cores": aff,
           "cpu_model": cpu_model(), "cpu_info": cpu_info(),
           "sample": (f"every kernel of the step (configs 2-4) and of config 5 at full shape on "
                      f"a host copy of buffer set 0; median of >= 10 runs after a warm-up, about "
                      f"{budget:.0f} s per thread count; oracle C restatement ({oracle_build()}, "
                      f"-O3, no FMA contraction, no fast-math), 1 thread and {n_all} "
                      f"OpenMP threads")}
    if ks70:
        c1, _ = rate(ks70, 1)
        cn, _ = rate(ks70, n_all)
        out["config5"] = {"value": cn, "cores": n_all, "single_thread_value": c1,
                          "unit": "GB/s"}
    return out


# --------------------------------------------------------------------------
# rocprof-derived traffic figure, if a committed summary exists
# --------------------------------------------------------------------------

def traffic_from_profiles(kernel, workload):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc
    summary of `workload` (profiles/<workload>_pmc.txt), if there is one."""
    path = os.path.join(ROOT, "profiles", f"{workload}_pmc.txt")
    if not os.path.exists(path):
        return None
    m = re.search(rf"^{re.escape(kernel)}_traffic_bytes_per_launch:\s*([0-9.]+)",
                  open(path).read(), re.M)
    return float(m.group(1)) if m else None


CALIB_BYTES = 256 << 20  # plain D2D copy used to scale the FETCH/WRITE counters


def calibrate_copy(torch, reps=5):
    """A plain device copy of known size (CALIB_BYTES read + written)."""
    src = torch.empty(CALIB_BYTES, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()


def clean_kernel(name):
    """Kernel name without its parameter list (templates kept)."""
    name = name.replace("(anonymous namespace)::", "")
    depth = 0
    for i, ch in enumerate(name):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            return name[:i]
    return name


def per_step_table(dbs, steps):
    """Every kernel of the run grouped by name: dispatches per step and GPU
    microseconds per step (sum of dispatch durations / steps)."""
    import sqlite3

    tot, setup = {}, 0.0
    for db in dbs:
        c = sqlite3.connect(db)
        for name, n, total in c.execute("select name, count(*), sum(duration) from kernels "
                                        "group by name"):
            k = clean_kernel(name)
            if "jinf::" not in k:  # torch's input generation and runtime copies
                setup += total
                continue
            a = tot.setdefault(k, [0, 0.0])
            a[0] += n
            a[1] += total
    all_us = sum(v[1] for v in tot.values()) / 1e3 / steps
    out = [f"per step ({steps} steps profiled; every dispatch of the library's kernels divided "
           f"by the step count): {all_us:.1f} us of kernel time per step",
           f"  {'kernel':72s} {'calls/step':>10s} {'us/step':>9s} {'share':>6s}"]
    for k, (n, total) in sorted(tot.items(), key=lambda kv: -kv[1][1]):
        us = total / 1e3 / steps
        out.append(f"  {k[:72]:72s} {n / steps:10.2f} {us:9.1f} {us / all_us:6.1%}")
    out.append(f"  (input generation and runtime copies outside the library: "
               f"{setup / 1e3:.0f} us in total, not per step)")
    return out


def rocprof_summary(dbs, bytes_per_kernel, steps=0):
    """Text summary of rocprofv3 databases: per-kernel dispatch durations and,
    for --pmc runs, per-dispatch FETCH_SIZE / WRITE_SIZE (KiB), the copy
    calibration factors, and the resulting HBM bytes per launch."""
    import sqlite3

    lines = []
    durs, ctrs = {}, {}
    for db in dbs:
        c = sqlite3.connect(db)
        # the copy calibration is the largest-grid blit; torch's small copies share its name
        big = c.execute("select max(grid_x * grid_y * grid_z) from kernels "
                        "where name like '%copyBuffer%'").fetchone()[0] or 0
        # the probes of several kernels share one kernel name: they are told
        # apart by their grid size (work-items)
        for name, gs, n, avg, mn, mx in c.execute(
                "select name, grid_x * grid_y * grid_z, count(*), avg(duration), min(duration), "
                "max(duration) from kernels where name not like '%copyBuffer%' "
                "or grid_x * grid_y * grid_z = ? group by name, grid_x, grid_y, grid_z", (big,)):
            key = probe_key(short_kernel(name), gs)
            if key:
                if key in durs:  # one key, several grids: merge (dispatch-weighted)
                    n0, a0, m0, x0 = durs[key]
                    durs[key] = (n0 + n, (a0 * n0 + avg * n) / (n0 + n), min(m0, mn), max(x0, mx))
                else:
                    durs[key] = (n, avg, mn, mx)
        try:
            rows = c.execute("select kernel_name, grid_size, counter_name, avg(value), count(*) "
                             "from counters_collection where kernel_name not like '%copyBuffer%' "
                             "or grid_size = ? group by kernel_name, grid_size, counter_name",
                             (big,)).fetchall()
        except sqlite3.OperationalError:
            rows = []
        for name, gs, cn, v, n in rows:
            key = probe_key(short_kernel(name), gs)
            if key:
                ctrs.setdefault((key, cn), (v, n))
    if steps:
        lines += per_step_table(dbs, steps)
    lines.append("kernel durations (rocprofv3 --kernel-trace), microseconds:")
    lines.append(f"  {'kernel':44s} {'calls':>6s} {'avg':>9s} {'min':>9s} {'max':>9s}")
    for k, (n, avg, mn, mx) in sorted(durs.items()):
        lines.append(f"  {k:44s} {n:6d} {avg / 1e3:9.3f} {mn / 1e3:9.3f} {mx / 1e3:9.3f}")
    if ctrs:
        lines.append("counters per dispatch (rocprofv3 --pmc), KiB:")
        for (k, cn), (v, n) in sorted(ctrs.items()):
            lines.append(f"  {k:44s} {cn:12s} {v:14.1f}  ({n} dispatches)")
        cal_f = ctrs.get(("copy_calibration", "FETCH_SIZE"))
        cal_w = ctrs.get(("copy_calibration", "WRITE_SIZE"))
        if cal_f and cal_w:
            ff = CALIB_BYTES / 1024 / cal_f[0]
            fw = CALIB_BYTES / 1024 / cal_w[0]
            lines.append(f"copy calibration ({CALIB_BYTES >> 20} MiB read + written): "
                         f"FETCH factor {ff:.4f}, WRITE factor {fw:.4f}")
            for k, nb in bytes_per_kernel.items():
                f = ctrs.get((k, "FETCH_SIZE"))
                w = ctrs.get((k, "WRITE_SIZE"))
                if f and w:
                    t = (f[0] * ff + w[0] * fw) * 1024
                    lines.append(f"{k}: traffic {t:.0f} B/launch vs algorithmic {nb} B "
                                 f"(ratio {t / nb:.3f})")
                    lines.append(f"{k}_traffic_bytes_per_launch: {t:.0f}")
    return "\n".join(lines)


_KERNEL_KEYS = [("ew_vec_kernel<unsigned short, 1", "swiglu"),
                ("ew_vec_kernel<unsigned short, 2", "residual_add_f16"),
                ("rmsnorm_vec_kernel<unsigned short, unsigned short, true", "residual_rmsnorm"),
                ("rmsnorm_vec_kernel", "rmsnorm"),
                ("embed_q4_0_kernel", "q4_0_gather"),
                ("rope_vec_kernel", "rope"),
                ("softmax_vec_kernel", "masked_softmax"),
                ("softmax_loop_kernel", "softmax_loop"),
                # the one-tile kernels serve q, k, v, o, gate, up; the multi-tile
                # kernels only down (14336 columns) in the GEMV workloads
                ("matvec_kernel<2, true, 0, 0,", "gemv_one_tile (q,k,v,o,gate,up)"),
                ("matvec_kernel<8, true, 0, 0,", "gemv_one_tile (q,k,v,o,gate,up)"),
                ("matvec_kernel<12, true, 0, 0,", "gemv_one_tile Q4_K (q,k,o,gate,up)"),
                ("matvec_kernel<14, true, 0, 0,", "gemv_one_tile Q6_K (v)"),
                ("matvec_kernel<2, false, 0, 0,", "gemv_down"),
                ("matvec_kernel<8, false, 0, 0,", "gemv_down"),
                ("matvec_kernel<12, false, 0, 0,", "gemv_down"),
                ("matvec_kernel<14, false, 0, 0,", "gemv_down"),
                ("matvec_any_kernel", "gemv_generic"),
                ("attn_decode_kernel", "gqa_attention"),
                ("attn_mfma_kernel", "gqa_attention"),
                ("attn_combine_kernel", "gqa_attention_combine"),
                ("attn_decode_any_kernel", "gqa_attention_generic"),
                ("copyBuffer", "copy_calibration"),
                ("probe_rows_inplace_kernel", "probe_rows_inplace"),
                ("probe_stream_kernel", "probe_stream"),
                ("probe_gather_kernel", "probe_gather"),
                ("probe_rows_ragged_kernel", "probe_rows_ragged"),
                ("probe_flat_kernel", "probe_flat"),
                ("am_clear_kernel", "attention counter clear"),
                # batched decode: matvec_batch_kernel<qtype, M-tiles, epilogue, tiles, waves, k-parts>
                ("matvec_batch_kernel<2, 1, 3,", "batch qkv+rope (Q4_0)"),
                ("matvec_batch_kernel<2, 1, 1,", "batch o/down+residual (Q4_0)"),
                ("matvec_batch_kernel<2, 1, 2,", "batch gate/up+swiglu (Q4_0)"),
                ("matvec_batch_kernel<14, 1, 0,", "batch output head (Q6_K)"),
                ("matvec_batch_kernel<2, 2, 3,", "batch qkv+rope (Q4_0, 2 M-tiles)"),
                ("matvec_batch_kernel<2, 2, 1,", "batch o/down+residual (Q4_0, 2 M-tiles)"),
                ("matvec_batch_kernel<2, 2, 2,", "batch gate/up+swiglu (Q4_0, 2 M-tiles)"),
                ("matvec_batch_kernel<14, 2, 0,", "batch output head (Q6_K, 2 M-tiles)"),
                ("matvec_batch_kernel", "batch gemv (other)"),
                ("mb_prepare_kernel", "batch x preparation"),
                ("mb_merge_kernel", "batch residual merge"),
                ("mb_qkv_epilogue_kernel", "batch qkv merge+rope"),
                ("bat_argmax", "batch argmax"),
                ("bat_begin_kernel", "batch step begin"),
                ("bat_embed", "batch embedding")]


def probe_key(key, grid_items):
    """Probe kernels are labelled with their grid size in work-items."""
    if key and key.startswith("probe"):
        return f"{key} [{grid_items} items]"
    return key


def short_kernel(name):
    for pat, key in _KERNEL_KEYS:
        if pat in name:
            return key
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="llama3-8b-layer")
    ap.add_argument("--batch", type=int, default=0,
                    help="sequences of llama3-8b-decode-batch (default 32, at most 64)")
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--prompt-tokens", type=int, default=512,
                    help="engine workloads: tokens of the timed prompt (0 = no prompt timing)")
    ap.add_argument("--cpu-seconds", type=float, default=20.0,
                    help="bounded CPU-baseline sample, split over the 1-thread and the "
                         "all-threads runs (0 = skip)")
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="threads of the all-cores CPU run (0 = the host cores this process "
                         "may use, at most 16: the GPU box's share for one GPU)")
    ap.add_argument("--kernel-launches", type=int, default=200,
                    help="back-to-back launches timed per kernel (at least --steps)")
    ap.add_argument("--no-ceilings", action="store_true",
                    help="skip the bandwidth-probe ceilings (counter-collection runs)")
    ap.add_argument("--no-config5", action="store_true",
                    help="default workload: skip the config-5 (70B decode chain) measurement")
    ap.add_argument("--no-graph", action="store_true",
                    help="launch eagerly instead of replaying a captured HIP graph")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a plain 256 MiB device copy (PMC scaling reference)")
    ap.add_argument("--rocprof-summary", nargs="+", metavar="DB",
                    help="summarize rocprofv3 result databases and exit (no GPU use)")
    ap.add_argument("--bytes", nargs="*", metavar="KERNEL=BYTES",
                    help="with --rocprof-summary: algorithmic bytes per launch of more kernels")
    ap.add_argument("--per-step", type=int, default=0, metavar="STEPS",
                    help="with --rocprof-summary: also every kernel's time per step, the run "
                         "holding STEPS steps")
    ap.add_argument("--no-f4", action="store_true",
                    help="default workload: skip the engine figures (batch-1 and batch-32 "
                         "decode of the Q4_0 Llama-3-8B-shaped model) and the GEMV and "
                         "attention figures (f1, f2)")
    ap.add_argument("--stream-curve", action="store_true",
                    help="print the geometry-free attainable stream rate per read:write mix "
                         "over transfer sizes 2-512 MB (a text table) and exit")
    args = ap.parse_args()

    if args.rocprof_summary:
        nb = {"rope": 10487808, "residual_rmsnorm": 67117056, "swiglu": 176160768,
              "q4_0_gather": 43008000, "gemv_down": 33103872}
        if args.bytes:  # extra "kernel=bytes" pairs (workloads with random shapes)
            for kv in args.bytes:
                k, v = kv.split("=")
                nb[k] = int(v)
        print(rocprof_summary(args.rocprof_summary, nb, args.per_step))
        return

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build measures one GPU only; the kernels are "
                          "row-independent and shard by rows with no exchange",
                          "n_gpus_requested": max(args.gpus, world)}), flush=True)
        sys.exit(2)

    import torch

    import jinf_amd

    jinf_amd.lib()
    torch.cuda.set_device(0)

    # The K timed steps are captured into one HIP graph and replayed once: the
    # GPU then runs the kernels back to back, as an engine's captured decode
    # step would, and Python launch overhead is out of the measurement.
    # --no-graph launches them eagerly on the stream instead.
    def record(n_steps, kernels, probe):
        for _ in range(n_steps):
            for k in kernels:
                k.run(probe)

    def timed(n_steps, kernels, probe=0):
        """GPU ms for n_steps passes over `kernels` (HIP events on the stream)."""
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        if args.no_graph:
            torch.cuda.synchronize()
            start.record()
            record(n_steps, kernels, probe)
            end.record()
        else:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                record(n_steps, kernels, probe)
            g.replay()  # untimed: first replay uploads the graph
            torch.cuda.synchronize()
            start.record()
            g.replay()
            end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end)

    log(f"{jinf_amd.version()} on {torch.cuda.get_device_name(0)}; workload {args.workload}")
    if args.stream_curve:
        print(stream_curve(torch, jinf_amd, timed, max(args.steps, args.kernel_launches)),
              flush=True)
        return
    if args.workload in ENGINE_MODELS:
        engine_bench(args, torch, jinf_amd)
        return
    ks, cfg, keep = workload(args.workload, torch, jinf_amd, args.seed)
    # the default run also measures config 5 (the 70B decode chain)
    ks70 = []
    if args.workload == "llama3-8b-layer" and not args.no_config5:
        g70 = torch.Generator(device="cuda")
        g70.manual_seed(args.seed)  # the same draw as --workload llama3-70b-decode
        ks70, cfg70 = config5(torch, jinf_amd, g70, keep)
    torch.cuda.synchronize()
    log("buffers ready: " + ", ".join(f"{k.name} x{len(k.launches)} sets"
                                      for k in ks + ks70))

    for _ in range(args.warmup):
        for k in ks + ks70:
            k.run()
            if k.probes and args.workload != "calibrate" and not args.no_ceilings:
                for u in k.probe_upls:
                    k.run(probe=u)
    torch.cuda.synchronize()

    t0 = time.perf_counter()
    total_ms = timed(args.steps, ks)
    wall = time.perf_counter() - t0
    chain_ms = timed(args.steps, ks70) / args.steps if ks70 else None
    # per-kernel average launch duration: each kernel alone, L launches back to
    # back over its rotating buffer sets, same event method; its probe likewise
    n_launch = max(args.steps, args.kernel_launches)
    for k in ks + ks70:
        k.ms = timed(n_launch, [k])
        k.n = n_launch
        if k.probes and args.workload != "calibrate" and not args.no_ceilings:
            # the ceiling: the fastest probe variant
            for u in k.probe_upls:
                ms = timed(n_launch, [k], probe=u)
                if k.ceil_ms is None or ms < k.ceil_ms:
                    k.ceil_ms, k.ceil_upl = ms, u
    # the geometry-free attainable rate of each kernel's mix at its size (after
    # every kernel is timed: these allocate and free their own buffer sets)
    if args.workload != "calibrate" and not args.no_ceilings:
        for k in ks + ks70:
            if k.name in KERNEL_MIX:
                k.att_us, k.att_lay = attainable(torch, jinf_amd, timed, KERNEL_MIX[k.name],
                                                 k.nbytes, n_launch)
    ms_step = total_ms / args.steps
    step_bytes = sum(k.nbytes for k in ks)
    kern_ms = sum(k.ms / k.n for k in ks)

    def per_kernel(kl, workload):
        per = {}
        for k in kl:
            us = k.ms / k.n * 1e3
            gbs = k.nbytes / (us * 1e-6) / 1e9
            e = {"us": round(us, 3), "GB/s": round(gbs, 1), "frac_of_8TBs": round(gbs / PEAK_GBS, 4),
                 "rows_per_s": round(k.rows / (us * 1e-6), 1), "row_unit": k.row_unit,
                 "bytes": k.nbytes, "sets": len(k.launches), "launches_timed": k.n}
            # ceiling: the faster of the probe in the kernel's own geometry
            # and the geometry-free attainable stream of its mix and size
            cus = None
            if k.ceil_ms is not None:
                cus = k.ceil_ms / k.n * 1e3
                e.update({"probe_us": round(cus, 3), "probe_frac": round(cus / us, 4),
                          "ceiling_probe": k.probe_name, "ceiling_units_per_lane": k.ceil_upl[0],
                          "ceiling_exchange": k.ceil_upl[1]})
            if getattr(k, "att_us", None) is not None:
                cus = k.att_us if cus is None else min(cus, k.att_us)
                e.update({"attainable_us": round(k.att_us, 3),
                          "attainable_frac": round(k.att_us / us, 4),
                          "attainable_mix": KERNEL_MIX[k.name],
                          "attainable_layout": list(k.att_lay)})
            if cus is not None:
                e.update({"ceiling_us": round(cus, 3),
                          "ceiling_GB/s": round(k.nbytes / (cus * 1e-6) / 1e9, 1),
                          "frac_of_ceiling": round(cus / us, 4)})
            t = traffic_from_profiles({"residual_add": "residual_add_f16"}.get(k.name, k.name),
                                      workload)
            if t is not None:
                e["traffic_bytes"] = t
                e["traffic_ratio"] = round(t / k.nbytes, 4)
            per[k.name] = e
        return per

    per = per_kernel(ks, args.workload)
    dom = max(ks, key=lambda k: k.ms)
    dom_us = dom.ms / dom.n * 1e3
    dom_gbs = dom.nbytes / (dom_us * 1e-6) / 1e9
    roofline = {"bound": "hbm", "kernel": dom.name, "hip_kernel": dom.hip_name,
                "achieved": round(dom_gbs, 1), "peak": PEAK_GBS, "unit": "GB/s",
                "frac": round(dom_gbs / PEAK_GBS, 4), "bytes_per_launch": dom.nbytes,
                "avg_launch_us": round(dom_us, 3), "launches_timed": dom.n,
                "traffic": traffic_from_profiles(dom.name, args.workload)}
    c5 = None
    if ks70:
        b70 = sum(k.nbytes for k in ks70)
        c5 = dict(cfg70, chain_us=round(chain_ms * 1e3, 3), chain_bytes=b70,
                  **{"chain_GB/s": round(b70 / (chain_ms * 1e-3) / 1e9, 1),
                     "chain_frac_of_8TBs": round(b70 / (chain_ms * 1e-3) / 1e9 / PEAK_GBS, 4)},
                  launch="HIP graph of the K chain steps, replayed once",
                  kernels=per_kernel(ks70, "llama3-70b-decode"))

    if args.calibrate_copy:
        calibrate_copy(torch)


    cpu = None
    if args.cpu_seconds > 0 and args.workload != "calibrate":
        try:
            cpu = cpu_baseline_both(ks, ks70, args)
        except Exception as exc:  # the baseline is reported, never required
            log(f"cpu baseline failed: {exc!r}")
            cpu = None

    # the engine rows, timed after the kernels (their buffers stay resident:
    # 288 GB of HBM holds both)
    f4 = None
    if args.workload == "llama3-8b-layer" and not args.no_f4:
        t0 = time.perf_counter()
        f4 = f4_figures(args, torch, jinf_amd)
        log(f"engine figures in {time.perf_counter() - t0:.1f} s: batch 1 "
            f"{f4['batch1']['ms_per_token']} ms/token, batch 32 "
            f"{f4['batch32']['ms_per_step']} ms/step")

    # the GEMV and attention rows: the seven batch-1 projections of
    # --workload llama3-8b-gemv (each beside the read-only stream of its bytes)
    # and the config-5-shaped decode attention of --workload
    # llama3-70b-attention, each kernel alone over its rotating sets as above
    f1 = f2 = None
    if args.workload == "llama3-8b-layer" and not args.no_f4:
        t0 = time.perf_counter()
        ksg, cfg_g, keep_g = workload("llama3-8b-gemv", torch, jinf_amd, args.seed)
        ksa, cfg_a, keep_a = workload("llama3-70b-attention", torch, jinf_amd, args.seed)
        for k in ksg + ksa:
            k.run()
        torch.cuda.synchronize()
        for k in ksg + ksa:
            k.ms = timed(n_launch, [k])
            k.n = n_launch
        if not args.no_ceilings:
            for k in ksg:
                k.att_us, k.att_lay = attainable(torch, jinf_amd, timed, KERNEL_MIX[k.name],
                                                 k.nbytes, n_launch)
        f1 = {"workload": cfg_g["workload"], "shapes": cfg_g["shapes"],
              "layer_us": round(sum(k.ms / k.n for k in ksg) * 1e3, 3),
              "kernels": per_kernel(ksg, "llama3-8b-gemv")}
        f2 = {"workload": cfg_a["workload"], "shapes": cfg_a["shapes"],
              "kernels": per_kernel(ksa, "llama3-70b-attention")}
        del ksg, ksa, keep_g, keep_a
        log(f"GEMV and attention figures in {time.perf_counter() - t0:.1f} s: seven batch-1 "
            f"GEMVs {f1['layer_us']} us, 70B-shape attention "
            f"{f2['kernels']['gqa_attention']['us']} us")

    out = {
        "metric": METRIC,
        "value": round(step_bytes / (ms_step * 1e-3) / 1e9, 1),
        "unit": "GB/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": cfg.pop("dtype", "f32 math, f16 storage"),
        "data": "synthetic: seeded torch RNG on device (N(mu, sigma), sigma = std); "
                "Q4_0 scales fp16(|N(0,0.02)|), nibbles uniform",
        "config": dict(cfg, step_bytes=step_bytes),
        "frac_of_peak": round(step_bytes / (ms_step * 1e-3) / 1e9 / PEAK_GBS, 4),
        "kernel_ms_per_step": round(kern_ms, 5),
        "launch": "eager stream" if args.no_graph else "HIP graph of the K steps, replayed once",
        "wall_s_timed": round(wall, 4),
        "kernels": per,
        "config5": c5,
        "f1": f1,
        "f2": f2,
        "f4": f4,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


def _cpuinfo_fields():
    f = {}
    try:
        for line in open("/proc/cpuinfo"):
            if ":" in line:
                k, v = line.split(":", 1)
                f.setdefault(k.strip(), []).append(v.strip())
    except OSError:
        pass
    return f


def cpu_model():
    f = _cpuinfo_fields()
    return f.get("model name", ["unknown"])[0]


def cpu_info():
    """Host CPU identification: /proc/cpuinfo fields and lscpu's summary."""
    f = _cpuinfo_fields()
    info = {k: f[k][0] for k in ("vendor_id", "model name", "cpu family", "model", "stepping",
                                 "cpu MHz", "cache size") if k in f}
    info["logical_cpus"] = len(f.get("processor", []))
    info["sockets"] = len(set(f.get("physical id", []))) or None
    try:
        import subprocess
        txt = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in txt.splitlines():
            k, _, v = line.partition(":")
            if k.strip() in ("Model name", "Socket(s)", "Core(s) per socket",
                             "Thread(s) per core", "CPU max MHz", "L3 cache"):
                info["lscpu " + k.strip()] = v.strip()
    except Exception:  # lscpu is optional
        pass
    return info


if __name__ == "__main__":
    main()
