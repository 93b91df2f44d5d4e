"""Benchmark of the MaxSim hot path on one MI355X; prints ONE JSON line.

Default workload (BASELINE metric): single-query MaxSim, Q[32,128] against
D[5000,300,128] fp16 (reference flash_maxsim(Q, D)), inputs resident in HBM.
A step is one flash_maxsim call over the whole batch. value = docs/s.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config NAME] [--rotate R] [--doc-align A] [--no-cpu]

Configs (the driver's line is the default, c1):
  c1         metric workload, config 1 at B = 5000
  c1_rot     the same with four distinct copies of D (1.5 GB) used in turn,
             so no step finds its docs in the 256 MB last-level cache
  c1_1000    config 1 at B = 1000 (its parity size)
  c1_topk    config 1 followed by top-100 selection (flash_maxsim_topk, one call)
  c1_torch_topk  config 1 followed by torch.topk(scores, 100): what callers do today
  c1_floor   config 1 followed by a one-element fill kernel: the cost of any
             dependent launch after scoring
  c2         config 2, visual: Q[1024,128] x D[1000,1024,128]
  c3         config 3, batched: Q[100,32,128] x D[5000,300,128], shared docs
  c3_zeros   config 3's shapes on all-zero Q and D: the same kernel and instruction
             stream with no bits toggling, to show what the power limit costs
  c3_pq      batched with per-query docs (shared_docs=False):
             Q[100,32,128] x D[100,50,300,128]
  c4         config 4, uint8 docs [5000,1024,128], lengths U[32,1024]
  c4_packed  config 4's docs in the packed layout
  c4_packed_sorted  the same, docs laid out longest first (sort_by_length)
  c4_lq128   config 4's docs against a 128-token query
  mid        the reference's published "medium" row: Q[128,128] x D[1000,1024,128]
  c5         config 5, training forward + backward, Q[128,1024] x D[1000,512,1024]
  quant      quantize_int8 of config 4's docs (fp16 source) on the GPU
  copy       a device copy of 384 MB, to calibrate HBM byte counters
--rotate R (R >= 2) cycles R copies of the doc tensor(s) for any config.
--doc-align A (c4_packed) starts each packed doc on a multiple of A token rows.
Any single-query shape: s_Lq_B_Ld_d (fp16 docs) or u8_Lq_B_Ld_d (quantize_int8
codes of the same random docs), e.g. s_32_5000_1024_128; several fp16 queries:
b_Nq_Lq_B_Ld_d (docs shared by all queries) or p_Nq_Lq_B_Ld_d (each query its own
B docs), e.g. p_100_32_1000_77_128.

roofline: the dominant kernel's algorithmic bytes (or flops) per launch divided
by its average launch duration, timed with HIP events recorded on the stream
the kernels run on (torch's current stream, which the library launches on).
cpu_baseline: the reference's CPU path, maxsim_naive in fp32 (plain torch on
the host, all threads this process may use), on a bounded sample of the same
workload (same fp16 values widened to fp32), repeated for about 10 s.
"""

from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0

METRIC = "MaxSim docs/sec + % HBM/MFMA roofline, Lq=32 Ld=300 d=128 B=5000 fp16"
CPU_SAMPLE_S = 10.0  # seconds of CPU baseline work


def sim(shape, seed, dtype, device="cpu"):
    """Reference input recipe: N(0,1) rows, L2-normalised per token, cast."""
    import torch

    g = torch.Generator().manual_seed(seed)
    x = torch.nn.functional.normalize(torch.randn(*shape, generator=g), dim=-1).to(dtype)
    return x.to(device)


def cpu_threads() -> int:
    """Host threads for the CPU baseline: the process's CPU share (OMP_NUM_THREADS
    when set, as on the GPU boxes), else the CPUs it may run on."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        return int(env)
    try:
        return max(1, len(os.sched_getaffinity(0)))
    except AttributeError:  # pragma: no cover
        return max(1, os.cpu_count() or 1)


class Workload:
    """One benchmark configuration.

    steps: callables, each one step of the hot path (several = the same work on
    rotated copies of the inputs); units: work units per step (docs, pairs);
    roof: {"bound", "amount" (bytes or flops per step), "unit", "kernel"};
    cpu_fn / cpu_units: the CPU baseline over a sample of `cpu_units` units.
    """

    def __init__(self, cfg, steps, units, unit, roof, cpu_fn=None, cpu_units=0, cpu_sample=""):
        self.cfg, self.steps, self.units, self.unit, self.roof = cfg, steps, units, unit, roof
        self.cpu_fn, self.cpu_units, self.cpu_sample = cpu_fn, cpu_units, cpu_sample


def _copies(t, rotate):
    """rotate distinct device copies of t (the first is t itself)."""
    return [t] + [t.clone() for _ in range(max(1, rotate) - 1)]


def _realign(packed, align: int):
    """The same packed docs with each doc's rows starting on a multiple of
    `align` token rows (gaps of zero rows between docs)."""
    import torch

    import flash_maxsim_amd as fm

    L = packed.lengths.to(torch.int64)
    n = (L + align - 1) // align * align
    start = torch.cumsum(n, 0) - n
    T = int(n.sum())
    j = torch.arange(int(L.max()), device=L.device)
    keep = j[None, :] < L[:, None]
    src = (4 * packed.tok_group[:, None] + j[None, :])[keep]
    dst = (start[:, None] + j[None, :])[keep]
    codes = torch.zeros(T, packed.codes.shape[1], dtype=packed.codes.dtype, device=L.device)
    scales = torch.zeros(T, dtype=packed.scales.dtype, device=L.device)
    mins = torch.zeros(T, dtype=packed.mins.dtype, device=L.device)
    codes[dst], scales[dst], mins[dst] = packed.codes[src], packed.scales[src], packed.mins[src]
    return fm.PackedInt8Docs(codes, scales, mins, (start // 4).contiguous(), packed.lengths, packed.max_len,
                             packed.doc_ids)


def build(name: str, rotate: int, doc_align: int = 4) -> Workload:
    import torch

    import flash_maxsim_amd as fm

    dev = "cuda"
    f16 = torch.float16

    if name in ("c1", "c1_rot", "c1_1000", "c1_topk", "c1_torch_topk", "c1_floor"):
        B = 1000 if name == "c1_1000" else 5000
        Lq, Ld, d, k = 32, 300, 128, 100
        if name == "c1_rot":
            rotate = max(rotate, 4)
        Q = sim((Lq, d), 11, f16)
        Dh = sim((B, Ld, d), 12, f16)
        Qd = Q.to(dev)
        Ds = _copies(Dh.to(dev), rotate)
        cfg = {"workload": f"single-query flash_maxsim Q[{Lq},{d}] x D[{B},{Ld},{d}] fp16", "B": B, "Lq": Lq,
               "Ld": Ld, "d": d}
        if rotate > 1:
            cfg["rotated_doc_copies"] = len(Ds)
        algo = B * Ld * d * 2 + Lq * d * 2 + B * 4
        Qc, Dc = Q.float(), Dh.float()
        if name == "c1_topk":
            cfg["workload"] = f"flash_maxsim_topk k={k}: " + cfg["workload"]
            cfg["k"] = k
            steps = [lambda D=D: fm.flash_maxsim_topk(Qd, D, k) for D in Ds]
            roof = {"bound": "hbm", "amount": algo + B * 4 + k * 12, "unit": "GB/s",
                    "kernel": "stream_fwd_kernel + topk"}
            cpu = lambda: torch.topk(fm.maxsim_naive(Qc, Dc), k)  # noqa: E731
            sample = f"maxsim_naive fp32 + torch.topk over all {B} docs"
        elif name == "c1_torch_topk":
            cfg["workload"] = f"flash_maxsim + torch.topk k={k}: " + cfg["workload"]
            cfg["k"] = k
            steps = [lambda D=D: torch.topk(fm.flash_maxsim(Qd, D), k) for D in Ds]
            roof = {"bound": "hbm", "amount": algo + B * 4 + k * 12, "unit": "GB/s",
                    "kernel": "stream_fwd_kernel + torch.topk"}
            cpu = lambda: torch.topk(fm.maxsim_naive(Qc, Dc), k)  # noqa: E731
            sample = f"maxsim_naive fp32 + torch.topk over all {B} docs"
        elif name == "c1_floor":
            cfg["workload"] = "flash_maxsim + a one-element fill kernel: " + cfg["workload"]
            one = torch.zeros(1, device=dev)
            steps = [lambda D=D: (fm.flash_maxsim(Qd, D), one.zero_()) for D in Ds]
            roof = {"bound": "hbm", "amount": algo, "unit": "GB/s", "kernel": "stream_fwd_kernel + fill"}
            cpu = lambda: fm.maxsim_naive(Qc, Dc)  # noqa: E731
            sample = f"maxsim_naive fp32 over all {B} docs"
        else:
            steps = [lambda D=D: fm.flash_maxsim(Qd, D) for D in Ds]
            roof = {"bound": "hbm", "amount": algo, "unit": "GB/s", "kernel": "stream_fwd_kernel"}
            cpu = lambda: fm.maxsim_naive(Qc, Dc)  # noqa: E731
            sample = f"maxsim_naive fp32 over all {B} docs"
        return Workload(cfg, steps, B, "docs/s", roof, cpu, B, sample)

    if name in ("c2", "mid"):
        B, Lq, Ld, d = 1000, (1024 if name == "c2" else 128), 1024, 128
        Q = sim((Lq, d), 21 if name == "c2" else 25, f16)
        Dh = sim((B, Ld, d), 22 if name == "c2" else 26, f16)
        Qd = Q.to(dev)
        Ds = _copies(Dh.to(dev), rotate)
        cfg = {"workload": f"single-query flash_maxsim Q[{Lq},{d}] x D[{B},{Ld},{d}] fp16", "B": B, "Lq": Lq,
               "Ld": Ld, "d": d}
        if rotate > 1:
            cfg["rotated_doc_copies"] = len(Ds)
        steps = [lambda D=D: fm.flash_maxsim(Qd, D) for D in Ds]
        if name == "c2":
            roof = {"bound": "mfma", "amount": 2 * Lq * Ld * d * B, "unit": "TFLOP/s", "kernel": "tiled_fwd_kernel"}
        else:
            roof = {"bound": "hbm", "amount": B * Ld * d * 2 + Lq * d * 2 + B * 4, "unit": "GB/s",
                    "kernel": "stream_fwd_kernel"}
        n = 100 if name == "c2" else 500
        Qc, Dc = Q.float(), Dh[:n].float()

        def cpu():
            for b0 in range(0, n, 50):  # chunks of 50 docs bound the similarity tensor
                fm.maxsim_naive(Qc, Dc[b0:b0 + 50])

        return Workload(cfg, steps, B, "docs/s", roof, cpu, n,
                        f"maxsim_naive fp32 over the first {n} docs in chunks of 50")

    if name in ("c3", "c3_pq", "c3_zeros"):
        Nq, Lq, Ld, d = 100, 32, 300, 128
        B = 50 if name == "c3_pq" else 5000
        Q = sim((Nq, Lq, d), 31, f16)
        shape = (Nq, B, Ld, d) if name == "c3_pq" else (B, Ld, d)
        Dh = sim(shape, 32 if name != "c3_pq" else 33, f16)
        if name == "c3_zeros":
            Q, Dh = torch.zeros_like(Q), torch.zeros_like(Dh)
        Qd = Q.to(dev)
        Ds = _copies(Dh.to(dev), rotate)
        shared = name != "c3_pq"
        desc = "shared docs" if shared else "per-query docs (shared_docs=False)"
        if name == "c3_zeros":
            desc += ", all-zero inputs"
        cfg = {"workload": f"batched flash_maxsim Q[{Nq},{Lq},{d}] x D{list(shape)} fp16 {desc}", "Nq": Nq,
               "B": B, "Lq": Lq, "Ld": Ld, "d": d}
        if rotate > 1:
            cfg["rotated_doc_copies"] = len(Ds)
        steps = [lambda D=D: fm.flash_maxsim_batched(Qd, D, None, shared) for D in Ds]
        if shared:
            roof = {"bound": "mfma", "amount": 2 * Nq * Lq * Ld * d * B, "unit": "TFLOP/s",
                    "kernel": "tiled_fwd_kernel"}
            n = 500
            Qc, Dc = Q.float(), Dh[:n].float()

            def cpu():  # per-query loop, as the reference benchmark runs its naive batched case
                for qi in range(Nq):
                    fm.maxsim_naive(Qc[qi], Dc)

            return Workload(cfg, steps, Nq * B, "pairs/s", roof, cpu, Nq * n,
                            f"maxsim_naive fp32, per-query loop over {Nq} queries x the first {n} docs")
        roof = {"bound": "hbm", "amount": Nq * B * Ld * d * 2 + Nq * Lq * d * 2 + Nq * B * 4, "unit": "GB/s",
                "kernel": "stream_fwd_kernel"}
        Qc, Dc = Q.float(), Dh.float()

        def cpu():
            for qi in range(Nq):
                fm.maxsim_naive(Qc[qi], Dc[qi])

        return Workload(cfg, steps, Nq * B, "pairs/s", roof, cpu, Nq * B,
                        f"maxsim_naive fp32, per-query loop over all {Nq} x {B} pairs")

    if name in ("c4", "c4_packed", "c4_packed_sorted", "c4_lq128"):
        B, Ld, d = 5000, 1024, 128
        Lq = 128 if name == "c4_lq128" else 32
        Q = sim((Lq, d), 41 if Lq == 32 else 45, f16)
        lengths = torch.randint(32, 1025, (B,), generator=torch.Generator().manual_seed(43), dtype=torch.int32)
        tot = int(lengths.sum())
        codes = torch.empty(B, Ld, d, dtype=torch.uint8, device=dev)
        scales = torch.empty(B, Ld, 1, dtype=f16, device=dev)
        mins = torch.empty(B, Ld, 1, dtype=f16, device=dev)
        for b0 in range(0, B, 500):  # quantize_int8 on the GPU: bit-identical to the torch formula
            x = sim((500, Ld, d), 42 + b0, torch.float32, dev)
            codes[b0:b0 + 500], scales[b0:b0 + 500], mins[b0:b0 + 500] = fm.quantize_int8(x)
            del x
        Qd, ld = Q.to(dev), lengths.to(dev)
        n = 300
        cc, cs, cm, cl = codes[:n].cpu(), scales[:n].cpu(), mins[:n].cpu(), lengths[:n]
        Qc = Q.float()
        cpu = lambda: fm.maxsim_naive(Qc, fm.dequantize_int8(cc, cs, cm), cl)  # noqa: E731
        sample = f"maxsim_naive fp32 against dequantize_int8 of the first {n} docs, with their lengths"
        if name in ("c4_packed", "c4_packed_sorted"):
            srt = name == "c4_packed_sorted"
            Dg = torch.empty(B, Ld, d, dtype=torch.float32, device=dev)
            for b0 in range(0, B, 500):
                Dg[b0:b0 + 500] = sim((500, Ld, d), 42 + b0, torch.float32, dev)
            packed = fm.quantize_int8_packed(Dg, lengths, sort_by_length=srt)
            del Dg, codes, scales, mins
            if doc_align > 4:
                packed = _realign(packed, doc_align)
            packs = [packed] + [fm.PackedInt8Docs(packed.codes.clone(), packed.scales.clone(), packed.mins.clone(),
                                                  packed.tok_group, packed.lengths, packed.max_len, packed.doc_ids)
                                for _ in range(max(1, rotate) - 1)]
            cfg = {"workload": f"int8 packed varlen flash_maxsim_int8_packed Q[{Lq},{d}] x {B} docs of "
                               f"U[32,1024] tokens, d={d} u8 ({packed.codes.shape[0]} packed rows"
                               f"{', longest first' if srt else ''})", "B": B,
                   "Lq": Lq, "d": d, "sum_len": tot}
            if doc_align > 4:
                cfg["doc_align_rows"] = doc_align
            steps = [lambda p=p: fm.flash_maxsim_int8_packed(Qd, p) for p in packs]
            algo = tot * (d + 4) + Lq * d * 2 + B * (20 if srt else 16)  # + tok_group, lengths, scores (, doc_ids)
        else:
            sets = [(codes, scales, mins)] + [(codes.clone(), scales.clone(), mins.clone())
                                              for _ in range(max(1, rotate) - 1)]
            cfg = {"workload": f"int8 fused-dequant varlen flash_maxsim_int8 Q[{Lq},{d}] x D[{B},{Ld},{d}] u8, "
                               f"len U[32,1024]", "B": B, "Lq": Lq, "Ld": Ld, "d": d, "sum_len": tot}
            steps = [lambda s=s: fm.flash_maxsim_int8(Qd, s[0], s[1], s[2], ld) for s in sets]
            algo = tot * (d + 4) + Lq * d * 2 + B * 8
        if rotate > 1:
            cfg["rotated_doc_copies"] = len(steps)
        kern = "stream_u8_shared_kernel" if name == "c4_lq128" else "stream_fwd_kernel"
        roof = {"bound": "hbm", "amount": algo, "unit": "GB/s", "kernel": kern}
        return Workload(cfg, steps, B, "docs/s", roof, cpu, n, sample)

    if name == "quant":
        B, Ld, d = 5000, 1024, 128
        Dg = torch.empty(B, Ld, d, dtype=f16, device=dev)
        for b0 in range(0, B, 500):
            Dg[b0:b0 + 500] = sim((500, Ld, d), 42 + b0, f16, dev)
        cfg = {"workload": f"quantize_int8 of D[{B},{Ld},{d}] fp16 -> u8 codes + fp16 scales/mins", "B": B,
               "Ld": Ld, "d": d}
        roof = {"bound": "hbm", "amount": B * Ld * (d * 2 + d + 4), "unit": "GB/s", "kernel": "quantize_kernel"}
        n = 100
        Dc = Dg[:n].cpu()
        return Workload(cfg, [lambda: fm.quantize_int8(Dg)], B, "docs/s", roof, lambda: fm.quantize_int8(Dc), n,
                        f"quantize_int8 (torch formula) on the CPU over the first {n} docs")

    if name == "c5":
        B, Lq, Ld, d = 1000, 128, 512, 1024
        Q = sim((Lq, d), 51, f16)
        Dh = sim((B, Ld, d), 52, f16)
        Qd = Q.to(dev).requires_grad_(True)
        Dds = [D.requires_grad_(True) for D in _copies(Dh.to(dev), rotate)]

        def make_step(Dd):
            def step():
                s = fm.flash_maxsim_train(Qd, Dd)
                s.sum().backward()
                Qd.grad = None
                Dd.grad = None
            return step

        cfg = {"workload": f"train fwd+bwd flash_maxsim_train Q[{Lq},{d}] x D[{B},{Ld},{d}] fp16", "B": B,
               "Lq": Lq, "Ld": Ld, "d": d}
        if rotate > 1:
            cfg["rotated_doc_copies"] = len(Dds)
        # D read by the forward + dD written + the B*Lq rows of D gathered for dQ
        # + argmax written and read back (Q, dQ and scores are < 1 MB).
        roof = {"bound": "hbm", "amount": 2 * B * Ld * d * 2 + B * Lq * d * 2 + B * Lq * 4 * 2, "unit": "GB/s",
                "kernel": "splitd_fwd_kernel + bwd kernels (whole step)"}
        n = 8
        Qc = Q.float().requires_grad_(True)
        Dc = Dh[:n].float().requires_grad_(True)

        def cpu():  # fp32 autograd through maxsim_naive, as the reference benchmark's naive training
            fm.maxsim_naive(Qc, Dc).sum().backward()
            Qc.grad = None
            Dc.grad = None

        return Workload(cfg, [make_step(D) for D in Dds], B, "docs/s", roof, cpu, n,
                        f"maxsim_naive fp32 forward + autograd backward over the first {n} docs")

    if name == "copy":
        n = 5000 * 300 * 128
        src = torch.empty(n, dtype=f16, device=dev).normal_()
        dst = torch.empty_like(src)
        cfg = {"workload": f"device copy of {n * 2} bytes (counter calibration)", "bytes": n * 2}
        roof = {"bound": "hbm", "amount": 2 * n * 2, "unit": "GB/s", "kernel": "copy"}
        return Workload(cfg, [lambda: dst.copy_(src)], 1, "copies/s", roof)

    shape = re.fullmatch(r"(s|u8)_(\d+)_(\d+)_(\d+)_(\d+)", name)
    if shape:  # any single-query shape: s_Lq_B_Ld_d (fp16) or u8_Lq_B_Ld_d (uint8 codes)
        kind = shape.group(1)
        Lq, B, Ld, d = map(int, shape.groups()[1:])
        Q = sim((Lq, d), 61, f16)
        Qd, Qc = Q.to(dev), Q.float()
        n = min(B, 200)
        if kind == "s":
            Dh = sim((B, Ld, d), 62, f16)
            Ds = _copies(Dh.to(dev), rotate)
            steps = [lambda D=D: fm.flash_maxsim(Qd, D) for D in Ds]
            Dc = Dh[:n].float()
            cpu = lambda: fm.maxsim_naive(Qc, Dc)  # noqa: E731
            amount, flops = B * Ld * d * 2 + Lq * d * 2 + B * 4, 2 * Lq * B * Ld * d
            what = "fp16"
        else:
            sets = []
            for _ in range(max(1, rotate)):
                x = sim((B, Ld, d), 62 + len(sets), torch.float32, dev)
                sets.append(fm.quantize_int8(x))
                del x
            steps = [lambda st=st: fm.flash_maxsim_int8(Qd, *st) for st in sets]
            cc, cs, cm = (t[:n].cpu() for t in sets[0])
            cpu = lambda: fm.maxsim_naive(Qc, fm.dequantize_int8(cc, cs, cm))  # noqa: E731
            amount, flops = B * Ld * (d + 4) + Lq * d * 2 + B * 4, 2 * Lq * B * Ld * d
            what = "u8"
        cfg = {"workload": f"single-query Q[{Lq},{d}] x D[{B},{Ld},{d}] {what}", "B": B, "Lq": Lq, "Ld": Ld, "d": d}
        if rotate > 1:
            cfg["rotated_doc_copies"] = len(steps)
        mfma = flops / MFMA_F16_PEAK_TFLOPS / 1e12 > amount / HBM_PEAK_GBS / 1e9
        roof = ({"bound": "mfma", "amount": flops, "unit": "TFLOP/s", "kernel": "forward"} if mfma else
                {"bound": "hbm", "amount": amount, "unit": "GB/s", "kernel": "forward"})
        return Workload(cfg, steps, B, "docs/s", roof, cpu, n, f"maxsim_naive fp32 over the first {n} docs")

    shape = re.fullmatch(r"(p|b)_(\d+)_(\d+)_(\d+)_(\d+)_(\d+)", name)
    if shape:  # several queries: p_ (per-query docs) or b_ (docs shared by all queries)
        kind = shape.group(1)
        Nq, Lq, B, Ld, d = map(int, shape.groups()[1:])
        Q = sim((Nq, Lq, d), 63, f16)
        Qd, Qc = Q.to(dev), Q.float()
        n = min(B, 50)
        nq = min(Nq, 4)
        if kind == "p":
            Dh = sim((Nq, B, Ld, d), 64, f16)
            Ds = _copies(Dh.to(dev), rotate)
            steps = [lambda D=D: fm.flash_maxsim_batched(Qd, D, None, False) for D in Ds]
            Dc = Dh[:nq, :n].float()
            cpu = lambda: [fm.maxsim_naive(Qc[i], Dc[i]) for i in range(nq)]  # noqa: E731
            amount = Nq * B * Ld * d * 2 + Nq * Lq * d * 2 + Nq * B * 4
            what, docs = "per-query docs", f"D[{Nq},{B},{Ld},{d}]"
        else:
            Dh = sim((B, Ld, d), 64, f16)
            Ds = _copies(Dh.to(dev), rotate)
            steps = [lambda D=D: fm.flash_maxsim_batched(Qd, D) for D in Ds]
            Dc = Dh[:n].float()
            cpu = lambda: [fm.maxsim_naive(Qc[i], Dc) for i in range(nq)]  # noqa: E731
            amount = B * Ld * d * 2 + Nq * Lq * d * 2 + Nq * B * 4
            what, docs = "shared docs", f"D[{B},{Ld},{d}]"
        flops = 2 * Nq * Lq * B * Ld * d
        cfg = {"workload": f"batched flash_maxsim Q[{Nq},{Lq},{d}] x {docs} fp16 {what}", "Nq": Nq, "B": B,
               "Lq": Lq, "Ld": Ld, "d": d}
        if rotate > 1:
            cfg["rotated_doc_copies"] = len(steps)
        mfma = flops / MFMA_F16_PEAK_TFLOPS / 1e12 > amount / HBM_PEAK_GBS / 1e9
        roof = ({"bound": "mfma", "amount": flops, "unit": "TFLOP/s", "kernel": "forward"} if mfma else
                {"bound": "hbm", "amount": amount, "unit": "GB/s", "kernel": "forward"})
        return Workload(cfg, steps, Nq * B, "pairs/s", roof, cpu, nq * n,
                        f"maxsim_naive fp32, {nq} queries x the first {n} docs")

    raise SystemExit(f"unknown config {name}")


def measured_traffic(config: str):
    """HBM bytes per launch of the dominant kernel, from the committed rocprofv3 --pmc
    summaries in profiles/ (line `traffic_bytes_per_launch[<config>] = N`), or None."""
    import re

    pat = re.compile(r"^traffic_bytes_per_launch\[" + re.escape(config) + r"\]\s*=\s*(\d+)", re.M)
    for f in sorted((ROOT / "profiles").glob("*.md")):
        m = pat.search(f.read_text())
        if m:
            return int(m.group(1)), f"profiles/{f.name}"
    return None, None


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # Default warmup runs ~20 ms of back-to-back launches: MFMA work on random data
    # sets off the GPU's power management for the first few ms of a sustained run
    # (launch time 66 -> ~85 -> 63 us at the metric shape), and the timed steps
    # should see the clocks the GPU settles at, not that transient.
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=300)
    ap.add_argument("--config", default="c1", help="workload name (see the module docstring)")
    ap.add_argument("--rotate", type=int, default=1, help="cycle this many copies of the docs")
    ap.add_argument("--doc-align", type=int, default=4,
                    help="c4_packed: start each packed doc on a multiple of this many token rows (4 = packed)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: every GPU box of this build has one MI355X; sharding docs "
              "across GPUs is a design here, not a run.", file=sys.stderr)
        raise SystemExit(2)

    import torch

    torch.cuda.set_device(0)
    if args.doc_align < 4 or args.doc_align % 4:
        raise SystemExit("--doc-align must be a positive multiple of 4")
    w = build(args.config, args.rotate, args.doc_align)
    steps = w.steps
    for i in range(args.warmup):
        steps[i % len(steps)]()
    torch.cuda.synchronize()

    # The library launches on torch's current stream; one event pair brackets the
    # whole timed region on that stream (per-step event records would put marker
    # packets, and GPU idle gaps, between back-to-back launches).
    stream = torch.cuda.current_stream()
    ev_start = torch.cuda.Event(enable_timing=True)
    ev_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev_start.record(stream)
    for i in range(args.steps):
        steps[i % len(steps)]()
    ev_end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1000.0 / args.steps
    kern_ms = ev_start.elapsed_time(ev_end) / args.steps  # average launch duration on the kernel's stream
    value = w.units / (ms_per_step / 1000.0)

    roof = w.roof
    achieved = roof["amount"] / (kern_ms / 1000.0)
    if roof["unit"] == "GB/s":
        achieved /= 1e9
        peak = HBM_PEAK_GBS
    else:
        achieved /= 1e12
        peak = MFMA_F16_PEAK_TFLOPS
    traffic, traffic_src = measured_traffic(args.config) if args.doc_align == 4 else (None, None)
    roofline = {"bound": roof["bound"], "achieved": round(achieved, 2), "peak": peak, "unit": roof["unit"],
                "frac": round(achieved / peak, 4), "traffic": traffic, "traffic_source": traffic_src,
                "algorithmic": roof["amount"], "kernel": roof["kernel"],
                "kernel_ms": round(kern_ms, 5)}

    cpu = None
    if not args.no_cpu and w.cpu_fn is not None:
        # Bounded sample: the reference's CPU path over `cpu_units` units of the
        # same workload, repeated until at least CPU_SAMPLE_S seconds have run.
        threads = cpu_threads()
        torch.set_num_threads(threads)
        with torch.inference_mode(args.config != "c5"):
            w.cpu_fn()  # warm
            calls = 0
            t = time.perf_counter()
            while True:
                w.cpu_fn()
                calls += 1
                el = time.perf_counter() - t
                if el >= CPU_SAMPLE_S and calls >= 3:
                    break
        what = w.unit.split("/")[0]
        cpu = {"value": round(w.cpu_units * calls / el, 2), "unit": w.unit, "cores": threads, "kind": "port",
               "sample": f"{calls} x {w.cpu_units} {what} ({el:.1f} s): {w.cpu_sample}, "
                         f"torch {torch.__version__} on {threads} threads, {cpu_model()}"}

    line = {
        "metric": METRIC if args.config == "c1" and args.rotate <= 1 else f"{args.config}: {w.cfg['workload']}",
        "value": round(value, 1),
        "unit": w.unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",  # MFMA operands (uint8 codes are widened to fp16 exactly), fp32 accumulation
        "data": "synthetic",
        "config": w.cfg,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
