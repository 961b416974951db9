#!/usr/bin/env python
"""Benchmark of the GPTQ hot path on one MI355X.

Workload (config 3): quantize one Llama-3-8B-shaped decoder block (hidden
4096, 32 query / 8 KV heads of 128, SwiGLU FFN 14336, bf16 random init) to
4-bit g128 with act-order, from 128 x 2048 calibration tokens.  A step =
block forward over all tokens collecting the four distinct layer inputs
(q/k/v, o, gate/up, down), four one-triangle Hessians, four damped
Cholesky/inverse factorisations, seven column sweeps with lazy-batch
updates, and packing of all seven layers.  Inputs (calibration activations
and weights) are resident in HBM before timing starts.

The JSON line also reports the Hessian kernel against the bf16 MFMA
roofline; config 4, the W4A16 / W3A16 dequant-GEMV/GEMM microbench (M = 1,
16, 128, rotating >= 1 GiB of distinct weight buffers so HBM, not the 256 MB
last-level cache, is measured) beside what a read-only launch of the same
bytes achieves; config 1 (one Linear(768, 768), s per layer), config 2 (the
OPT-125m-shaped model) and config 5 (the 13B-shaped model at 4-bit g128
act-order, one pass and block by block), each wall time and peak HBM; and a
CPU baseline: the CPU oracle on this host's cores, config 1 and config 4's
fallback forward in full, the block extrapolated from measured samples.

    python bench.py [--steps 3] [--warmup 1] [--no-cpu] [--no-gemv] [--no-models]
    python bench.py --workload opt125m     # config 2 alone
    python bench.py --workload llama13b    # config 5 alone, 2/4/8 bits
    python bench.py --workload kernels     # the kernel set the counter summaries cover
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "s per 8B-shaped block quantized; Hessian MFMA TFLOP/s; W4A16 GEMV HBM GB/s"
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0
# Bytes moved below the L2 by the down_proj Hessian's tile + reduce launches
# (the roofline's kernel, run alone over 262144 tokens), from two rocprofv3
# counter passes over this script (FETCH_SIZE, then WRITE_SIZE), calibrated
# against the hipMemcpy copies of known size in the same runs
# (profiles/hessian_llama8b_block_traffic.md).
HESSIAN_TRAFFIC = {"tokens": 262144, "read": 91.61e9, "written": 2.50e9}

HID, NQ, NKV, HD, FFN = 4096, 32, 8, 128, 14336


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ------------------------------------------------------------ the block --

class Block:
    """Random-init Llama-3-8B-shaped decoder block (bf16)."""

    def __init__(self, torch, dev, seed=2):
        g = torch.Generator(device=dev).manual_seed(seed)

        def w(n, k):
            return (torch.randn(n, k, generator=g, device=dev, dtype=torch.float32) * 0.02).to(torch.bfloat16)

        self.w = {"q_proj": w(NQ * HD, HID), "k_proj": w(NKV * HD, HID), "v_proj": w(NKV * HD, HID),
                  "o_proj": w(HID, NQ * HD), "gate_proj": w(FFN, HID), "up_proj": w(FFN, HID),
                  "down_proj": w(HID, FFN)}
        gamma = torch.ones(HID, device=dev, dtype=torch.float32)
        idx = torch.randperm(HID, generator=g, device=dev)[:8]
        gamma[idx] = 20.0
        self.g1 = gamma.to(torch.bfloat16)
        self.g2 = torch.ones(HID, device=dev, dtype=torch.bfloat16)
        self.hkey = {"q_proj": "qkv", "k_proj": "qkv", "v_proj": "qkv", "o_proj": "o", "gate_proj": "up",
                     "up_proj": "up", "down_proj": "down"}

        # fused q/k/v projection for the forward (the GPTQ layers stay separate);
        # gate and up stay two products so that SiLU and the product run on
        # contiguous tensors (on column slices of one fused output they take
        # torch's strided elementwise path)
        self.wqkv = torch.cat([self.w["q_proj"], self.w["k_proj"], self.w["v_proj"]], 0)
        self.gqa = None

    @staticmethod
    def rmsnorm_into(torch, F, x, gamma, out, eps=1e-5):
        torch.mul(F.rms_norm(x, (x.shape[-1],), eps=eps), gamma, out=out)

    def rope(self, torch, T, dev):
        inv = 1.0 / (500000.0 ** (torch.arange(0, HD, 2, device=dev, dtype=torch.float32) / HD))
        t = torch.arange(T, device=dev, dtype=torch.float32)
        f = torch.outer(t, inv)  # both halves of a head share these angles
        return f.cos().to(torch.bfloat16), f.sin().to(torch.bfloat16)

    @staticmethod
    def apply_rope(torch, x, cos, sin):
        """rotate-half RoPE; x (..., T, heads, HD), cos/sin (T, 1, HD/2)"""
        x1, x2 = x[..., : HD // 2], x[..., HD // 2:]
        out = torch.empty(x.shape, device=x.device, dtype=x.dtype)
        o1, o2 = out[..., : HD // 2], out[..., HD // 2:]
        torch.mul(x1, cos, out=o1)
        o1.addcmul_(x2, sin, value=-1)
        torch.mul(x2, cos, out=o2)
        o2.addcmul_(x1, sin)
        return out

    def attention(self, torch, F, q, k, v):
        """causal SDPA, flash/efficient kernels; grouped KV heads natively
        when the backend takes them, else repeated"""
        from torch.nn.attention import SDPBackend, sdpa_kernel
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            if self.gqa is None:
                try:
                    F.scaled_dot_product_attention(q[:1, :, :16], k[:1, :, :16], v[:1, :, :16], is_causal=True,
                                                   enable_gqa=True)
                    self.gqa = True
                except Exception:  # noqa: BLE001 -- backend without grouped heads
                    self.gqa = False
            if self.gqa:
                return F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)
            k = k.repeat_interleave(NQ // NKV, dim=1)
            v = v.repeat_interleave(NQ // NKV, dim=1)
            return F.scaled_dot_product_attention(q, k, v, is_causal=True)

    def collect(self, torch, F, z, bufs, chunk, cos, sin, seqs=None):
        """Forward over sequences [s_begin, s_end) (all by default); store the
        four layer inputs (written in place into their calibration buffers)."""
        nseq, T, _ = z.shape
        c, s_ = cos[:, None], sin[:, None]
        s_begin, s_end = seqs if seqs is not None else (0, nseq)
        for s0 in range(s_begin, s_end, chunk):
            zc = z[s0:s0 + chunk]
            b = zc.shape[0]
            r0, r1 = s0 * T, (s0 + b) * T
            x1 = bufs["qkv"][r0:r1].view(b, T, HID)
            self.rmsnorm_into(torch, F, zc, self.g1, x1)
            qkv = F.linear(x1, self.wqkv).view(b, T, NQ + 2 * NKV, HD)
            qk = self.apply_rope(torch, qkv[:, :, : NQ + NKV], c, s_)
            q = qk[:, :, :NQ].transpose(1, 2)
            k = qk[:, :, NQ:].transpose(1, 2)
            v = qkv[:, :, NQ + NKV:].transpose(1, 2)
            a = self.attention(torch, F, q, k, v)
            o_in = bufs["o"][r0:r1].view(b, T, NQ, HD)
            o_in.copy_(a.transpose(1, 2))
            h = torch.add(zc, F.linear(o_in.view(b, T, HID), self.w["o_proj"]))
            x2 = bufs["up"][r0:r1].view(b, T, HID)
            self.rmsnorm_into(torch, F, h, self.g2, x2)
            g_ = F.silu(F.linear(x2, self.w["gate_proj"]), inplace=True)
            torch.mul(g_, F.linear(x2, self.w["up_proj"]), out=bufs["down"][r0:r1].view(b, T, FFN))


def hessian_flops(n, K):
    """one triangle incl. the diagonal, 2 flops per multiply-add"""
    return n * K * (K + 1)


def run_block(args, torch, F, dev):
    from distributed_gptq_amd import _ops, pipeline
    blk = Block(torch, dev)
    T, nseq = args.seqlen, args.nseq
    n = nseq * T
    g = torch.Generator(device=dev).manual_seed(2)
    z = torch.randn(nseq, T, HID, generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    bufs = {k: torch.empty(n, HID if k != "down" else FFN, device=dev, dtype=torch.bfloat16)
            for k in ("qkv", "o", "up", "down")}
    Hs = {k: torch.empty(v.shape[1], v.shape[1], device=dev, dtype=torch.float32) for k, v in bufs.items()}
    cos, sin = blk.rope(torch, T, dev)
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731

    # The forward runs in `groups` groups of sequences; each group's four
    # Hessian accumulations go to a dedicated stream while the next group's
    # forward runs on the main stream (H += X_g^T X_g, the reference's
    # per-batch add_batch).  The down_proj chain (largest K) is the critical
    # path: after the last group its Hessian is finished first and its
    # factorisation / sweep start on a side stream, then the other three
    # Hessians finish and their chains start on three more side streams.
    # Three side streams plus the main stream fill the 4 hardware queues HIP
    # uses by default (a fifth stream would share a queue and serialise): the
    # down_proj chain, the gate/up chain, the q/k/v chain, and the o_proj
    # chain on the main stream after the Hessians.
    pool = pipeline.side_streams(dev, 4)
    G = max(1, min(args.hessian_groups, nseq))
    # one group: the Hessians follow the forward on the main stream
    hst, pool = (pool[3] if G > 1 else torch.cuda.current_stream(dev)), pool[:3]
    first = "down"
    order = [first] + [k for k in Hs if k != first]
    names = {k: [n for n in blk.w if blk.hkey[n] == k] for k in Hs}
    bounds = [(g * nseq // G, (g + 1) * nseq // G) for g in range(G)]

    def step(record):
        e = [ev() for _ in range(4)]
        he = {k: [] for k in Hs}
        main = torch.cuda.current_stream(dev)
        e[0].record()

        def start(keys, streams):
            w = {n: blk.w[n] for k in keys for n in names[k]}
            return pipeline.quantize_layers_async(w, blk.hkey, {k: (Hs[k], nseq) for k in keys}, bits=args.bits,
                                                  group_size=128, blocksize=128, percdamp=0.01, actorder=True,
                                                  want_dequant=True, check=True, streams=streams)

        hst.wait_stream(main)  # the previous step's chains have read H
        with torch.cuda.stream(hst):
            for k in order:
                Hs[k].zero_()
        p_first = p_rest = None
        for gi, (s0, s1) in enumerate(bounds):
            blk.collect(torch, F, z, bufs, args.chunk, cos, sin, seqs=(s0, s1))
            hst.wait_stream(main)
            last = gi == G - 1
            if last:
                e[1].record()
            with torch.cuda.stream(hst):
                for k in order:
                    a, b = ev(), ev()
                    a.record()
                    _ops.hessian_accumulate(Hs[k], bufs[k][s0 * T:s1 * T])
                    b.record()
                    he[k].append((a, b))
                    if last and k == first:
                        p_first = start([first], pool[:1])
                if last:
                    e[2].record()
                    p_rest = start(order[1:], [pool[1], pool[2], hst])
        main.wait_stream(hst)
        done = {**p_first.wait(), **p_rest.wait()}
        res = {n: done[n] for n in blk.w}
        e[3].record()
        if record is not None:
            torch.cuda.synchronize()
            record.append({
                "forward_ms": e[0].elapsed_time(e[1]),
                "hessian_ms": e[1].elapsed_time(e[2]),
                "quantize_ms": e[2].elapsed_time(e[3]),
                "hessian_kernel_ms": {k: sum(a.elapsed_time(b) for a, b in he[k]) for k in he},
            })
        return res

    for _ in range(args.warmup):
        step(None)
    torch.cuda.synchronize()
    recs = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        res = step(recs)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    s_per_block = wall / args.steps
    hflops = sum(hessian_flops(n, X.shape[1]) for X in bufs.values())
    # X read once, H read and written once
    hbytes = sum(n * X.shape[1] * 2 + 2 * X.shape[1] ** 2 * 4 for X in bufs.values())
    Ks = {k: X.shape[1] for k, X in bufs.items()}
    hms = sum(sum(r["hessian_kernel_ms"].values()) for r in recs) / len(recs)
    per_kernel = {k: sum(r["hessian_kernel_ms"][k] for r in recs) / len(recs) for k in Hs}
    breakdown = {k: round(sum(r[k] for r in recs) / len(recs), 3) for k in ("forward_ms", "hessian_ms", "quantize_ms")}
    losses = {k: float(v.losses_sum.item()) for k, v in res.items()}
    # the dominant kernel alone: the down_proj Hessian over all tokens (the
    # block's own calibration data), timed on its stream: the mean of three
    # launch pairs after one untimed
    iso = []
    for i in range(4):
        a, b = ev(), ev()
        Hs[first].zero_()
        a.record()
        _ops.hessian_accumulate(Hs[first], bufs[first])
        b.record()
        torch.cuda.synchronize()
        if i:
            iso.append(a.elapsed_time(b))
    iso_ms = sum(iso) / len(iso)
    iso_flops = hessian_flops(n, bufs[first].shape[1])
    iso_bytes = n * bufs[first].shape[1] * 2 + 2 * bufs[first].shape[1] ** 2 * 4
    del bufs, Hs, z
    torch.cuda.empty_cache()
    return dict(s_per_block=s_per_block, wall=wall, hessian_flops=hflops, hessian_bytes=hbytes, hessian_ms=hms,
                hessian_iso_ms=iso_ms, hessian_iso_flops=iso_flops, hessian_iso_bytes=iso_bytes, groups=G,
                hessian_kernel_ms=per_kernel, breakdown=breakdown, tokens=n, losses=losses,
                hessian_tflops_by_key={k: hessian_flops(n, Hs_k) / (per_kernel[k] * 1e-3) / 1e12
                                       for k, Hs_k in Ks.items()},
                attention="sdpa, grouped KV heads" if blk.gqa else "sdpa, KV heads repeated")


# ------------------------------------------------------------ GEMV bench --

GEMV_SHAPES = [(4096, 4096), (14336, 4096), (4096, 14336), (28672, 4096)]


def gemv_bytes(N, K, bits, M=1):
    return N * K * bits // 8 + N * (K // 128) * 4 + M * K * 2 + M * N * 2


def run_gemv(args, torch, dev, bits, M=1, min_bytes=1 << 30, reps=3, actorder=False):
    """Per-launch time of gptq_linear (act-order: gptq_linear_perm, weights
    stored in sweep order and x gathered through a random permutation) at
    the config-4 shapes, inside a HIP graph, rotating >= 1 GiB of weights."""
    from distributed_gptq_amd import _ops
    out = {}
    g = torch.Generator(device=dev).manual_seed(3)
    for (N, K) in GEMV_SHAPES:
        nbytes = gemv_bytes(N, K, bits, M) + (K * 4 if actorder else 0)
        R = max(2, math.ceil(min_bytes / (N * K * bits // 8)))
        codes = torch.randint(0, 2 ** bits, (N, K), generator=g, device=dev, dtype=torch.uint8)
        q0 = _ops.pack(codes, bits)
        qs = [q0.clone() for _ in range(R)]
        sc = [(torch.rand(N, K // 128, generator=g, device=dev) * 9e-3 + 1e-3).half() for _ in range(R)]
        zr = torch.full((N, K // 128), float(2 ** (bits - 1)), device=dev, dtype=torch.float16)
        x = torch.randn(M, K, generator=g, device=dev, dtype=torch.float32).half()
        y = torch.empty(M, N, device=dev, dtype=torch.float16)
        perm = torch.randperm(K, generator=g, device=dev).to(torch.int32) if actorder else None
        graph = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for r in range(R):  # warm-up (and the workspace of this stream) outside the capture
                _ops.linear(x, qs[r], bits, sc[r], zr, K, group_size=128, out=y, perm=perm)
            s.synchronize()
            with torch.cuda.graph(graph, stream=s):
                for r in range(R):
                    _ops.linear(x, qs[r], bits, sc[r], zr, K, group_size=128, out=y, perm=perm)
        torch.cuda.current_stream().wait_stream(s)
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (reps * R)
        out[f"{N}x{K}"] = {"us": round(us, 3), "GBps": round(nbytes / us * 1e-3, 1), "bytes": nbytes, "buffers": R}
        if M > 1:
            out[f"{N}x{K}"]["TFLOPs"] = round(2.0 * M * N * K / us * 1e-6, 1)
        del qs, sc, graph
        torch.cuda.empty_cache()
    tot_b = sum(v["bytes"] for v in out.values())
    tot_us = sum(v["us"] for v in out.values())
    return out, tot_b / tot_us * 1e-3


def run_fused(args, torch, dev, bits=4, M=1, min_bytes=1 << 30, reps=3):
    """Layers that share an input, as a decode step runs them: Llama-3-8B's
    q/k/v (4096 + 1024 + 1024 rows) and gate/up (2 x 14336 rows) over K =
    4096, once as separate gptq_linear launches and once as one launch over
    the concatenated rows (FusedQuantizedLinear), inside a HIP graph,
    rotating >= 1 GiB of weights."""
    from distributed_gptq_amd import _ops
    K = HID
    out = {}
    g = torch.Generator(device=dev).manual_seed(5)
    for name, rows in (("qkv", [NQ * HD, NKV * HD, NKV * HD]), ("gate_up", [FFN, FFN])):
        N = sum(rows)
        nbytes = gemv_bytes(N, K, bits, M)
        R = max(2, math.ceil(min_bytes / (N * K * bits // 8)))
        codes = torch.randint(0, 2 ** bits, (N, K), generator=g, device=dev, dtype=torch.uint8)
        q0 = _ops.pack(codes, bits)
        qs = [q0.clone() for _ in range(R)]
        sc = [(torch.rand(N, K // 128, generator=g, device=dev) * 9e-3 + 1e-3).half() for _ in range(R)]
        zr = torch.full((N, K // 128), float(2 ** (bits - 1)), device=dev, dtype=torch.float16)
        x = torch.randn(M, K, generator=g, device=dev, dtype=torch.float32).half()
        y = torch.empty(M, N, device=dev, dtype=torch.float16)
        offs = [sum(rows[:i]) for i in range(len(rows))]
        # separate layers: row slices of the same buffers (contiguous views)
        parts = [[(q[o:o + n], s_[o:o + n], zr[o:o + n], torch.empty(M, n, device=dev, dtype=torch.float16))
                  for o, n in zip(offs, rows)] for q, s_ in zip(qs, sc)]
        res = {}
        for mode in ("separate", "fused"):
            def body(r):
                if mode == "fused":
                    _ops.linear(x, qs[r], bits, sc[r], zr, K, group_size=128, out=y)
                else:
                    for (qp, sp, zp, yp) in parts[r]:
                        _ops.linear(x, qp, bits, sp, zp, K, group_size=128, out=yp)
            graph = torch.cuda.CUDAGraph()
            st = torch.cuda.Stream()
            st.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(st):
                for r in range(R):
                    body(r)
                st.synchronize()
                with torch.cuda.graph(graph, stream=st):
                    for r in range(R):
                        body(r)
            torch.cuda.current_stream().wait_stream(st)
            graph.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                graph.replay()
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / (reps * R)
            res[mode] = {"us": round(us, 3), "GBps": round(nbytes / us * 1e-3, 1), "launches": 1 if mode == "fused"
                         else len(rows)}
            del graph
        res["rows"] = rows
        res["bytes"] = nbytes
        out[name] = res
        del qs, sc, parts
        torch.cuda.empty_cache()
    return out


def run_read_ceiling(torch, dev, min_bytes=1 << 30, reps=3):
    """What one launch can read: gptq_stream_read (16-byte non-temporal loads,
    grid-stride) over each config-4 shape's W4A16 M = 1 byte count, in a HIP
    graph rotating >= 1 GiB of distinct buffers like the GEMV rows; best of
    5 grid sizes x 4 unroll depths."""
    import ctypes

    from distributed_gptq_amd import _lib
    lib = _lib.lib()
    out = {}
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    for (N, K) in GEMV_SHAPES:
        nbytes = gemv_bytes(N, K, 4, 1)
        pitch = (nbytes + 255) // 256 * 256
        R = max(2, math.ceil(min_bytes / nbytes))
        buf = torch.randint(0, 255, (R * pitch,), device=dev, dtype=torch.uint8)
        best = None
        for blocks in (256, 512, 1024, 2048, 4096):
            for unroll in (1, 2, 4, 8):
                def body():
                    st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
                    for r in range(R):
                        _lib.check(lib.gptq_stream_read(ctypes.c_void_p(buf.data_ptr() + r * pitch), nbytes,
                                                        blocks, unroll, ctypes.c_void_p(flag.data_ptr()), st),
                                   "gptq_stream_read")
                s = torch.cuda.Stream(device=dev)
                s.wait_stream(torch.cuda.current_stream(dev))
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.stream(s):
                    body()
                    s.synchronize()
                    with torch.cuda.graph(graph, stream=s):
                        body()
                torch.cuda.current_stream(dev).wait_stream(s)
                graph.replay()
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(reps):
                    graph.replay()
                e1.record()
                torch.cuda.synchronize()
                us = e0.elapsed_time(e1) * 1e3 / (reps * R)
                if best is None or us < best["us"]:
                    best = {"us": round(us, 3), "GBps": round(nbytes / us * 1e-3, 1), "bytes": nbytes,
                            "blocks": blocks, "unroll": unroll, "buffers": R}
                del graph
        out[f"{N}x{K}"] = best
        del buf
        torch.cuda.empty_cache()
    return out


def run_c1(torch, dev, reps=3):
    """Config 1 on the GPU: GPTQ of Linear(768, 768) (fp32, W ~ N(0, 0.02^2),
    seed 0) from 128 add_batch calls of (1, 512, 768) fp32 tokens with 8
    outlier channels x 20, 4-bit g128, to packed codes: reference mode
    (GPTQ.quantize + GPTQ.pack_weights, core/gptq.py:63-266) and canonical
    mode (GPTQ.fasterquant + the packed int32 QuantizedLinear).  Inputs are
    resident on the GPU; one warm-up, then the median of ``reps`` runs, each
    phase closed by a device synchronisation."""
    from distributed_gptq_amd import GPTQ
    from distributed_gptq_amd.models.layers import QuantizedLinear
    g = torch.Generator().manual_seed(0)
    W = torch.randn(768, 768, generator=g) * 0.02
    X = torch.randn(128, 512, 768, generator=g)
    X[..., torch.randperm(768, generator=g)[:8]] *= 20
    Wd, Xd = W.to(dev), X.to(dev)

    def once(mode):
        lin = torch.nn.Linear(768, 768).to(dev)
        with torch.no_grad():
            lin.weight.copy_(Wd)
            lin.bias.zero_()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        q = GPTQ(lin, bits=4, group_size=128, blocksize=128, percdamp=0.01, device=dev)
        for i in range(128):
            q.add_batch(Xd[i:i + 1])
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        if mode == "reference":
            q.quantize()
        else:
            q.fasterquant()
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        if mode == "reference":
            q.pack_weights()
        else:
            QuantizedLinear.from_gptq(q)
        torch.cuda.synchronize()
        t3 = time.perf_counter()
        return {"s": t3 - t0, "add_batch_s": t1 - t0, "quantize_s": t2 - t1, "pack_s": t3 - t2}

    out = {}
    for mode in ("reference", "canonical"):
        once(mode)
        runs = sorted((once(mode) for _ in range(reps)), key=lambda r: r["s"])
        med = runs[len(runs) // 2]
        out[mode] = {k: round(v, 5) for k, v in med.items()}
    out["note"] = ("s per layer, add_batch x 128 to packed codes; median of 3 after one warm-up; "
                   "reference = GPTQ.quantize + pack_weights, canonical = fasterquant + packed QuantizedLinear")
    return out


# ------------------------------------------------------------ CPU baseline --

def _host_cpu():
    """CPU model, physical / logical cores and the cores this process may use."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        import psutil
        physical = psutil.cpu_count(logical=False)
    except Exception:  # noqa: BLE001 -- psutil missing or restricted
        physical = None
    return {"cpu_model": model, "physical_cores": physical, "logical_cores": os.cpu_count(),
            "affinity_cores": len(os.sched_getaffinity(0))}


def _timed_cpu(fn, reps=1):
    """Median wall time of ``reps`` calls (after one warm-up when reps > 1)."""
    if reps > 1:
        fn()
    ts = []
    for _ in range(reps):
        t = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t)
    return sorted(ts)[len(ts) // 2]


BLOCK_LAYERS = [("q_proj", 4096, 4096), ("k_proj", 1024, 4096), ("v_proj", 1024, 4096), ("o_proj", 4096, 4096),
                ("gate_proj", 14336, 4096), ("up_proj", 14336, 4096), ("down_proj", 4096, 14336)]


def cpu_baseline():
    """The CPU oracle (numpy, this host's BLAS threads) as the reference
    computes, phase by phase (add_batch; damp + inverse; column sweep; pack):

    * config 1 in full (768 x 768, 128 x 512 fp32 tokens), reference mode
      (core/gptq.py:63-266 with the repair at :175) and canonical mode, one
      warm-up then the median of 3;
    * the config-3 block (128 x 2048 tokens), extrapolated per Linear from
      measured samples: reference mode for the layers it defines (N <= K:
      q/k/v/o/down), canonical mode for gate/up (N > K); one full-square
      Hessian per Linear, as the reference accumulates it;
    * config 4's fallback forward (models/layers.py:98-138, 155-157): the
      fp32 dequantisation of the codes then F.linear in fp32, at the four
      shapes and M = 1, 16, 128, measured in full."""
    import numpy as np
    from threadpoolctl import threadpool_info
    from oracle import gptq_oracle as O
    threads = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    rng = np.random.default_rng(0)
    t_all = time.perf_counter()

    # -- config 1, in full
    W1 = (rng.standard_normal((768, 768)) * 0.02).astype(np.float32)
    X1 = rng.standard_normal((128, 512, 768), dtype=np.float32)
    X1[..., rng.permutation(768)[:8]] *= 20
    c1 = {}
    for mode in ("reference", "canonical"):
        ph = {}

        def run(mode=mode, ph=ph):
            t = time.perf_counter()
            H, ns = None, 0
            for i in range(128):
                H, ns = O.add_batch(H, ns, X1[i:i + 1], dtype=np.float32)
            t1 = time.perf_counter()
            if mode == "reference":
                Hinv = O.full_inverse(O.damp_ref(H, ns, 0.01))
                t2 = time.perf_counter()
                r = O.gptq_ref(W1, Hinv, 4, 128, 128)
                t3 = time.perf_counter()
                O.ref_pack_weights(r["codes"].astype(np.uint8), 4)
            else:
                Hc, dead = O.prepare_canonical_H(H, ns, 0.01)
                U = O.upper_chol_of_inverse(Hc)
                t2 = time.perf_counter()
                r = O.gptq_canonical(W1, H, ns, 4, 128, 128, 0.01, dtype=np.float32, U=U)
                t3 = time.perf_counter()
                O.pack_bitstream(r["codes"].astype(np.uint8), 4)
            t4 = time.perf_counter()
            ph.setdefault("runs", []).append({"add_batch_s": t1 - t, "damp_inverse_s": t2 - t1, "sweep_s": t3 - t2,
                                              "pack_s": t4 - t3, "s": t4 - t})
        for _ in range(4):
            run()
        runs = sorted(ph["runs"][1:], key=lambda r: r["s"])
        c1[mode] = {k: round(v, 4) for k, v in runs[1].items()}

    # -- config 3, samples at K = 4096 (fp32)
    K = 4096
    x = rng.standard_normal((2, 2048, K), dtype=np.float32)
    t_h = _timed_cpu(lambda: O.add_batch(None, 0, x, dtype=np.float32)) / 2          # per sequence
    H = (x.reshape(-1, K).T @ x.reshape(-1, K)).astype(np.float32)
    Hd = O.damp_ref(H, 2, 0.01).astype(np.float32)
    t_inv = _timed_cpu(lambda: O.full_inverse(Hd))                                 # reference: full inverse
    t_U = _timed_cpu(lambda: O.upper_chol_of_inverse(Hd))                          # canonical: upper factor
    Hinv = O.full_inverse(Hd).astype(np.float32)
    Wr = (rng.standard_normal((1024, K)) * 0.02).astype(np.float32)
    t_rs = _timed_cpu(lambda: O.gptq_ref(Wr, Hinv, 4, 128, 128))                   # 1024 columns x K rows
    Wc = (rng.standard_normal((4096, 1024)) * 0.02).astype(np.float32)
    Hs = H[:1024, :1024].copy()
    t_cs = _timed_cpu(lambda: O.gptq_canonical(Wc, Hs, 2, 4, 128, 128, 0.01, actorder=True, dtype=np.float32))
    codes = rng.integers(0, 16, (4096, 4096)).astype(np.uint8)
    t_rp = _timed_cpu(lambda: O.ref_pack_weights(codes, 4))
    t_cp = _timed_cpu(lambda: O.pack_bitstream(codes, 4))
    per_layer = {}
    for name, N, Kl in BLOCK_LAYERS:
        ref = N <= Kl
        hs = 128 * t_h * (Kl / K) ** 2
        inv = (t_inv if ref else t_U) * (Kl / K) ** 3
        sw = t_rs * (N / 1024) * (Kl / K) if ref else t_cs * (N / 4096) * (Kl / 1024) ** 2
        pk = (t_rp if ref else t_cp) * (N / 4096) * (Kl / 4096)
        per_layer[name] = {"mode": "reference" if ref else "canonical", "add_batch_s": round(hs, 2),
                           "damp_inverse_s": round(inv, 2), "sweep_s": round(sw, 2), "pack_s": round(pk, 3)}
    phases = {k: round(sum(v[k] for v in per_layer.values()), 2)
              for k in ("add_batch_s", "damp_inverse_s", "sweep_s", "pack_s")}
    total = sum(phases.values())

    # -- config 4's fallback forward, measured in full
    c4 = {}
    for (N, Kc) in GEMV_SHAPES:
        q = rng.integers(0, 16, (N, Kc)).astype(np.uint8)
        sc = rng.uniform(1e-3, 1e-2, (N, Kc // 128)).astype(np.float16)
        zr = np.full((N, Kc // 128), 8.0, np.float16)
        gi = np.arange(Kc) // 128
        t = time.perf_counter()
        Wd = O.dequant(q, sc, zr, gi)
        t_un = time.perf_counter() - t
        row = {"unpack_weights_s": round(t_un, 4)}
        for M in (1, 16, 128):
            xm = rng.standard_normal((M, Kc)).astype(np.float32)
            row[f"linear_m{M}_s"] = round(_timed_cpu(lambda xm=xm, Wd=Wd: xm @ Wd.T, 3), 5)
        c4[f"{N}x{Kc}"] = row
        del Wd, q

    return {"value": round(total, 2), "unit": "s/block", "cores": threads, "kind": "port",
            "host": _host_cpu(),
            "mode": ("reference mode (core/gptq.py semantics, repaired at :175) for q/k/v/o/down, canonical for "
                     "gate/up (N > K, which the reference cannot run); oracle in numpy fp32"),
            "sample": ("config 3 extrapolated per Linear from measured samples at K = 4096: add_batch of 2 x 2048 "
                       "tokens (x 128 sequences x (K/4096)^2, one full-square H per Linear as the reference "
                       "accumulates it), the damped full inverse / upper factor (x (K/4096)^3), the reference "
                       "sweep of 1024 columns x 4096 rows (x N/1024 x K/4096) and the canonical act-order sweep "
                       "of 4096 x 1024 (x N/4096 x (K/1024)^2), the 4096 x 4096 pack (x N K / 4096^2); config 1 "
                       "and config 4's fallback forward measured in full"),
            "measured": ["c1", "c4_fallback", "samples"], "extrapolated": ["value", "block_phases_s", "per_layer"],
            "block_phases_s": phases, "per_layer": per_layer,
            "samples_s": {"add_batch_per_seq_4096": round(t_h, 4), "full_inverse_4096": round(t_inv, 3),
                          "upper_factor_4096": round(t_U, 3), "ref_sweep_1024x4096": round(t_rs, 3),
                          "canonical_sweep_4096x1024": round(t_cs, 3), "ref_pack_4096x4096": round(t_rp, 4),
                          "pack_4096x4096": round(t_cp, 4)},
            "c1": c1, "c4_fallback": c4, "wall_s": round(time.perf_counter() - t_all, 1)}


# ------------------------------------------------- kernel set for counters --

def run_kernels(args, torch, dev):
    """The kernels the hardware-counter summaries cover, each launched a few
    times eagerly (no graphs, so every dispatch is profiled): a device copy
    of 512 MiB (the FETCH_SIZE / WRITE_SIZE calibration), the down_proj
    Hessian of the config-3 block (262144 bf16 tokens, K = 14336), the
    factorisation and 4-bit act-order sweep of a 4096 x 14336 layer, and the
    W4A16 GEMV / dequant-GEMM at the config-4 shapes for M = 1, 16, 128
    (8 distinct weight buffers per shape, so that weights come from HBM)."""
    from distributed_gptq_amd import _ops, pipeline
    out = {}

    def timed(fn, reps):
        ts = []
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1))
        return round(min(ts), 4)

    src = torch.empty(512 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    out["copy_512MiB_ms"] = timed(lambda: dst.copy_(src), 3)
    del dst
    # the read-only launch at the largest W4A16 M = 1 byte count (28672 x 4096)
    import ctypes

    from distributed_gptq_amd import _lib
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    nb = gemv_bytes(28672, 4096, 4, 1)

    def read():
        st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        for r in range(8):
            _lib.check(_lib.lib().gptq_stream_read(ctypes.c_void_p(src.data_ptr() + r * (64 << 20)), nb, 2048, 4,
                                                   ctypes.c_void_p(flag.data_ptr()), st), "gptq_stream_read")
    out["stream_read_62MB_us"] = round(timed(read, 3) * 1e3 / 8, 2)
    del src
    g = torch.Generator(device=dev).manual_seed(5)
    n, K = args.nseq * args.seqlen, FFN
    X = torch.randn(n, K, generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    H = torch.zeros(K, K, device=dev)
    out["hessian_ms"] = timed(lambda: _ops.hessian_accumulate(H, X), 3)
    out["hessian_tflops"] = round(hessian_flops(n, K) / (out["hessian_ms"] * 1e-3) / 1e12, 1)
    del X
    W = (torch.randn(HID, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    t0 = time.perf_counter()
    pipeline.quantize_layers({"down_proj": W}, {"down_proj": "down"}, {"down": (H, args.nseq)}, bits=4,
                             group_size=128, actorder=True, want_dequant=False)
    torch.cuda.synchronize()
    out["factor_sweep_s"] = round(time.perf_counter() - t0, 4)
    del W, H
    torch.cuda.empty_cache()
    for (N, Kg) in GEMV_SHAPES:
        codes = torch.randint(0, 16, (N, Kg), generator=g, device=dev, dtype=torch.uint8)
        qs = [_ops.pack(codes, 4) for _ in range(8)]
        sc = (torch.rand(N, Kg // 128, generator=g, device=dev) * 9e-3 + 1e-3).half()
        zr = torch.full((N, Kg // 128), 8.0, device=dev, dtype=torch.float16)
        for M in (1, 16, 128):
            x = torch.randn(M, Kg, generator=g, device=dev).half()

            def run(x=x):
                for q in qs:
                    _ops.linear(x, q, 4, sc, zr, Kg, group_size=128)
            out[f"w4a16_{N}x{Kg}_m{M}_us"] = round(timed(run, 2) * 1e3 / len(qs), 2)
        del qs, codes
        torch.cuda.empty_cache()
    return out


# ------------------------------------------------ whole-model workloads --
# Config 2 (OPT-125m shape) and config 5 (13B shape): random-init models built
# from transformers' architectures, calibrated on uniform random token ids and
# quantized layer by layer by DistributedGPTQuantizer.quantize_model (the
# reference's core/quantizer.py:79-165 flow: calibration forward with hooks,
# then every decoder Linear).  lm_head is not quantized (N > K: the
# reference's quantize() cannot run it).
MODELS = {
    "opt125m": {"arch": "opt", "layers": 12, "hidden": 768, "heads": 12, "ffn": 3072, "vocab": 50272,
                "nseq": 128, "seed": 1, "chunk": 16, "runs": [(4, 128, False)]},
    "llama13b": {"arch": "llama", "layers": 40, "hidden": 5120, "heads": 40, "ffn": 13824, "vocab": 32000,
                 "nseq": 256, "seed": 4, "chunk": 8, "runs": [(2, 64, True), (4, 128, True), (8, -1, True)]},
}


def build_model(spec, torch, dev):
    """Random-init fp16 model of the named shape, weights ~N(0, 0.02^2)."""
    from transformers import LlamaConfig, LlamaForCausalLM, OPTConfig, OPTForCausalLM
    torch.manual_seed(spec["seed"])
    if spec["arch"] == "opt":
        cfg = OPTConfig(vocab_size=spec["vocab"], hidden_size=spec["hidden"], num_hidden_layers=spec["layers"],
                        ffn_dim=spec["ffn"], num_attention_heads=spec["heads"], max_position_embeddings=2048,
                        word_embed_proj_dim=spec["hidden"], init_std=0.02, use_cache=False)
        cls = OPTForCausalLM
    else:
        cfg = LlamaConfig(vocab_size=spec["vocab"], hidden_size=spec["hidden"], intermediate_size=spec["ffn"],
                          num_hidden_layers=spec["layers"], num_attention_heads=spec["heads"],
                          num_key_value_heads=spec["heads"], max_position_embeddings=2048,
                          initializer_range=0.02, use_cache=False)
        cls = LlamaForCausalLM
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.float16)
    try:
        with torch.device(dev):
            model = cls(cfg)
    finally:
        torch.set_default_dtype(prev)
    return model.eval()


def decoder_linears(model, torch):
    """Every nn.Linear inside the decoder layers (lm_head excluded)."""
    return [n for n, m in model.named_modules() if isinstance(m, torch.nn.Linear) and ".layers." in n]


def run_model(args, torch, dev):
    chosen = [r for r in MODELS[args.workload]["runs"] if not args.model_bits or r[0] in args.model_bits]
    if not chosen:
        raise SystemExit(f"--model-bits {args.model_bits}: no run of {args.workload} has those bits")
    return _run_model(torch, dev, args.workload, chosen, args.warmup, args.true_sequential, args.model_nseq,
                      args.model_chunk, args.seqlen)


def _run_model(torch, dev, workload, chosen, warmup, true_sequential, nseq=0, chunk=0, seqlen=2048, base=None):
    """Whole-model quantization (``DistributedGPTQuantizer.quantize_model``)
    of the named shape for each (bits, group size, act-order) in ``chosen``,
    each on a fresh copy of the model, after ``warmup`` untimed runs of the
    first.  Returns the result dict and the base model (for reuse)."""
    import copy

    from distributed_gptq_amd import DistributedGPTQuantizer, QuantizationConfig
    spec = MODELS[workload]
    nseq = nseq or spec["nseq"]
    if base is None:
        log(f"[bench] {workload}: building the random-init model")
        base = build_model(spec, torch, dev)
    names = decoder_linears(base, torch)
    g = torch.Generator(device=dev).manual_seed(spec["seed"])
    ids = torch.randint(0, spec["vocab"], (nseq, seqlen), device=dev, generator=g)
    chunk = chunk or spec["chunk"]
    data = [ids[i:i + chunk] for i in range(0, nseq, chunk)]
    runs = []
    # untimed warm-up runs of the first setting (library initialisation, GEMM heuristics)
    settings = [chosen[0]] * warmup + list(chosen)
    for idx, (bits, gs, actorder) in enumerate(settings):
        timed = idx >= warmup
        model = copy.deepcopy(base)
        cfg = QuantizationConfig(bits=bits, group_size=gs, actorder=actorder, calibration_samples=nseq,
                                 true_sequential=true_sequential)
        dq = DistributedGPTQuantizer(cfg)
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        free0, total = torch.cuda.mem_get_info()
        t0 = time.perf_counter()
        def progress(done, total, name, stats):
            if done % 28 == 0 or done == total:
                log(f"[bench]   {done}/{total} layers quantized ({time.perf_counter() - t0:.1f} s)")

        dq.quantize_model(model, data, layers_to_quantize=names, progress_callback=progress)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        free1, _ = torch.cuda.mem_get_info()
        errs = dq.quantization_errors
        r = {"bits": bits, "group_size": gs, "actorder": actorder, "true_sequential": true_sequential,
             "wall_s": round(wall, 3),
             "layers": len(errs), "peak_allocated_GiB": round(torch.cuda.max_memory_allocated() / 2**30, 2),
             "device_used_GiB_after": round((total - free1) / 2**30, 2),
             "total_error": float(sum(errs.values()))}
        log(f"[bench] {workload} w{bits} g{gs}{'' if timed else ' (warm-up)'}: {r}")
        if timed:
            runs.append(r)
        del model, dq
        torch.cuda.empty_cache()
    return {"runs": runs, "nseq": nseq, "layers": len(names), "chunk": chunk,
            "params_GiB": round(sum(p.numel() for p in base.parameters()) * 2 / 2**30, 2)}, base


def _c2(torch, dev):
    """Config 2: the OPT-125m-shaped model, 4-bit g128, one warm-up run."""
    m, _ = _run_model(torch, dev, "opt125m", MODELS["opt125m"]["runs"], 1, False)
    return {"unit": "s/model", "workload": "opt125m", "nseq": m["nseq"], "quantized_linears": m["layers"],
            **m["runs"][0]}


def _c5(torch, dev):
    """Config 5: the 13B-shaped model, 4-bit g128 act-order, one pass and
    block by block (true-sequential), no warm-up run of its own (the block,
    GEMV and config-2 runs before it have initialised the library)."""
    m1, base = _run_model(torch, dev, "llama13b", [(4, 128, True)], 0, False)
    m2, _ = _run_model(torch, dev, "llama13b", [(4, 128, True)], 0, True, base=base)
    del base
    return {"unit": "s/model", "workload": "llama13b", "nseq": m1["nseq"], "quantized_linears": m1["layers"],
            "params_GiB": m1["params_GiB"], "one_pass": m1["runs"][0], "true_sequential": m2["runs"][0],
            "other_settings": "2-bit g64 and 8-bit per-channel: bench.py --workload llama13b"}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--bits", type=int, default=4)
    ap.add_argument("--nseq", type=int, default=128)
    ap.add_argument("--seqlen", type=int, default=2048)
    ap.add_argument("--chunk", type=int, default=16, help="sequences per forward chunk")
    ap.add_argument("--hessian-groups", type=int, default=1,
                    help="forward groups whose Hessian accumulation overlaps the next group's forward")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-gemv", action="store_true")
    ap.add_argument("--no-block", action="store_true")
    ap.add_argument("--no-models", action="store_true", help="skip configs 1, 2 and 5 in the default run")
    ap.add_argument("--no-3bit", action="store_true", help="skip the 3-bit block run")
    ap.add_argument("--workload", choices=["block", "kernels", *MODELS], default="block",
                    help="block: config 3 (default); opt125m: config 2; llama13b: config 5")
    ap.add_argument("--model-nseq", type=int, default=0, help="calibration sequences for a model workload")
    ap.add_argument("--model-bits", type=lambda v: [int(b) for b in v.split(",")], default=None,
                    help="only the runs of a model workload with these code widths (comma list)")
    ap.add_argument("--true-sequential", action="store_true",
                    help="model workloads: quantize block by block (QuantizationConfig.true_sequential)")
    ap.add_argument("--model-chunk", type=int, default=0, help="sequences per calibration forward (model workloads)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build quantizes on a single MI355X "
              "(no collectives or sharded path); run it with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    import torch.nn.functional as F
    dev = torch.device("cuda", 0)
    import distributed_gptq_amd  # noqa: F401
    from distributed_gptq_amd import _lib
    _lib.load()
    if args.workload == "kernels":
        print(json.dumps({"workload": "kernels (the set the counter summaries cover)",
                          **run_kernels(args, torch, dev)}), flush=True)
        return
    if args.workload != "block":
        m, _ = run_model(args, torch, dev)
        spec = MODELS[args.workload]
        first = m["runs"][0]
        print(json.dumps({
            "metric": f"s per {args.workload}-shaped model quantized (calibration forward + Hessians + every decoder Linear)",
            "value": first["wall_s"], "unit": "s/model", "n_gpus": 1, "steps": 1, "warmup": args.warmup,
            "ms_per_step": round(first["wall_s"] * 1e3, 1), "higher_is_better": False, "scaling": "weak",
            "vs_baseline": None, "dtype": "fp16",
            "data": "synthetic (random-init weights N(0,0.02^2), uniform random token ids)",
            "config": {"workload": args.workload, "layers": spec["layers"], "hidden": spec["hidden"],
                       "heads": spec["heads"], "ffn": spec["ffn"], "vocab": spec["vocab"], "nseq": m["nseq"],
                       "seq_len": args.seqlen, "sequences_per_forward": m["chunk"],
                       "quantized_linears": m["layers"], "params_GiB": m["params_GiB"],
                       "parallelism": "single-gpu"},
            "runs": m["runs"]}), flush=True)
        return
    result = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
              "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
              "data": "synthetic (random-init weights, N(0,1) calibration with RMSNorm outlier channels)",
              "config": {"workload": f"llama3-8b-block-w{args.bits}g128-actorder", "hidden": HID, "heads": NQ,
                         "kv_heads": NKV, "ffn": FFN, "tokens": args.nseq * args.seqlen, "bits": args.bits,
                         "group_size": 128, "blocksize": 128, "percdamp": 0.01, "actorder": True,
                         "parallelism": "single-gpu"}}
    if not args.no_block:
        log(f"[bench] block: {args.nseq} x {args.seqlen} tokens, warmup {args.warmup}, steps {args.steps}")
        b = run_block(args, torch, F, dev)
        tflops_blk = b["hessian_flops"] / (b["hessian_ms"] * 1e-3) / 1e12
        tflops = b["hessian_iso_flops"] / (b["hessian_iso_ms"] * 1e-3) / 1e12
        result.update({"value": round(b["s_per_block"], 4), "unit": "s/block",
                       "ms_per_step": round(b["s_per_block"] * 1e3, 2),
                       "hessian_groups": b["groups"], "breakdown_ms": b["breakdown"],
                       "hessian_tflops_in_block": round(tflops_blk, 1),
                       "hessian_kernel_ms_in_block": {k: round(v, 3) for k, v in b["hessian_kernel_ms"].items()},
                       "layer_losses": {k: round(v, 4) for k, v in b["losses"].items()}})
        result["roofline"] = {"bound": "mfma", "kernel": "hessian_gram16 + hessian_reduce (down_proj input, alone)",
                              "achieved": round(tflops, 1), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                              "frac": round(tflops / PEAK_BF16_TFLOPS, 4), "traffic": None,
                              "launch_ms": round(b["hessian_iso_ms"], 3),
                              "work": f"n*K*(K+1) flops, n = {args.nseq * args.seqlen} tokens, K = {FFN}"}
        if args.nseq * args.seqlen == HESSIAN_TRAFFIC["tokens"] and HESSIAN_TRAFFIC["read"] is not None:
            t = HESSIAN_TRAFFIC
            result["roofline"].update({
                "traffic": round(t["read"] + t["written"]),
                "traffic_scope": "bytes per tile + reduce launch pair, below the L2 (MALL hits included)",
                "algorithmic_bytes": round(b["hessian_iso_bytes"])})
        result["config"]["forward_attention"] = b["attention"]
        if args.bits == 4 and not args.no_3bit:
            # the same block at 3 bits (g128, act-order): a second configuration of the workload
            a3 = argparse.Namespace(**{**vars(args), "bits": 3, "steps": max(1, min(args.steps, 2))})
            b3 = run_block(a3, torch, F, dev)
            result["block_3bit"] = {"s_per_block": round(b3["s_per_block"], 4), "breakdown_ms": b3["breakdown"],
                                    "layer_losses": {k: round(v, 4) for k, v in b3["losses"].items()}}
            log(f"[bench] 3-bit block: {b3['s_per_block']:.3f} s/block, {b3['breakdown']}")
        log(f"[bench] block done: {b['s_per_block']:.3f} s/block, groups {b['groups']}, {b['breakdown']}, "
            f"Hessian in block {tflops_blk:.1f} TFLOP/s, down_proj Hessian alone {tflops:.1f} TFLOP/s, "
            f"{b['attention']}")
    if not args.no_gemv:
        g4, agg4 = run_gemv(args, torch, dev, 4)
        log(f"[bench] W4A16 GEMV: {g4}")
        g3, agg3 = run_gemv(args, torch, dev, 3)
        log(f"[bench] W3A16 GEMV: {g3}")
        result["w4a16_gemv_gbps"] = round(agg4, 1)
        result["w3a16_gemv_gbps"] = round(agg3, 1)
        result["gemv"] = {"w4a16_m1": g4, "w3a16_m1": g3, "peak_GBps": PEAK_HBM_GBS,
                          "w4a16_frac": round(agg4 / PEAK_HBM_GBS, 4)}
        # batched activations (the dequant-GEMM path), M = 16 and 128
        for bits in (4, 3):
            for M in (16, 128):
                gm, _ = run_gemv(args, torch, dev, bits, M=M)
                result["gemv"][f"w{bits}a16_m{M}"] = gm
                log(f"[bench] W{bits}A16 M={M}: {gm}")
        # act-order layers (GPTQ output with act-order, the block's own
        # setting): sweep-order storage, x gathered through the permutation
        for M in (1, 16, 128):
            gm, _ = run_gemv(args, torch, dev, 4, M=M, actorder=True)
            result["gemv"][f"w4a16_actorder_m{M}"] = gm
            log(f"[bench] W4A16 act-order M={M}: {gm}")
        # layers sharing an input in one launch (decode step, M = 1)
        fu = run_fused(args, torch, dev)
        result["gemv"]["w4a16_m1_shared_input"] = fu
        log(f"[bench] W4A16 M=1 shared-input layers, separate vs one launch: {fu}")
        # what one launch of the same bytes can read, and the GEMV against it
        ceil = run_read_ceiling(torch, dev)
        result["gemv"]["read_ceiling"] = ceil
        result["gemv"]["w4a16_m1_frac_of_read_ceiling"] = {
            k: round(ceil[k]["us"] / g4[k]["us"], 4) for k in ceil}
        log(f"[bench] read-only launch at the W4A16 M=1 byte counts: {ceil}")
    if not args.no_models:
        # configs 1, 2 and 5 (each guarded: one failing run leaves the others' results)
        for key, fn in (("c1", lambda: run_c1(torch, dev)), ("c2", lambda: _c2(torch, dev)),
                        ("c5", lambda: _c5(torch, dev))):
            try:
                result[key] = fn()
                log(f"[bench] {key}: {result[key]}")
            except Exception as e:  # noqa: BLE001 -- recorded in the JSON line instead of losing it
                result[key] = {"error": f"{type(e).__name__}: {e}"}
                log(f"[bench] {key} failed: {e}")
            torch.cuda.empty_cache()
    if args.no_block:
        result.setdefault("value", None)
    if not args.no_cpu:
        log("[bench] CPU baseline (oracle on host cores)")
        result["cpu_baseline"] = cpu_baseline()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
