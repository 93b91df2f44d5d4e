"""Benchmark of the MaxSim hot path on one MI355X; prints ONE JSON line.

Default workload (BASELINE metric): single-query MaxSim, Q[32,128] against
D[5000,300,128] fp16 (reference flash_maxsim(Q, D)), inputs resident in HBM.
A step is one flash_maxsim call over the whole batch. value = docs/s.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
                    [--config c1|c1_1000|c1_topk|c2|c3|c4|c4_packed|quant|c5|copy]

The other configs are the remaining BASELINE configs (c2-c5), config 1 with
top-100 selection (c1_topk), config 4 over packed docs (c4_packed), the GPU
quantiser on config 4's docs (quant) and a
device copy for counter calibration (copy), for measurement runs; the
driver's line is the default (c1).

roofline: the dominant kernel's algorithmic bytes (or flops) per launch divided
by its average launch duration, timed with HIP events recorded on the stream
the kernel runs on (torch's current stream, which the library launches on).
cpu_baseline: the CPU oracle (oracle/, float64 accumulation, all host cores)
timed on the same workload.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0

METRIC = "MaxSim docs/sec + % HBM/MFMA roofline, Lq=32 Ld=300 d=128 B=5000 fp16"
CPU_SAMPLE_S = 10.0  # seconds of CPU oracle work behind cpu_baseline


def sim(shape, seed, dtype):
    import torch

    g = torch.Generator().manual_seed(seed)
    return torch.nn.functional.normalize(torch.randn(*shape, generator=g), dim=-1).to(dtype)


def make_workload(name):
    """Returns (description dict, step callable, work units per step, roofline spec, oracle sample fn)."""
    import numpy as np
    import torch

    import flash_maxsim_amd as fm
    import oracle

    dev = "cuda"
    if name in ("c1", "c1_1000"):
        B = 5000 if name == "c1" else 1000
        Lq, Ld, d = 32, 300, 128
        Q = sim((Lq, d), 11, torch.float16)
        Dh = sim((B, Ld, d), 12, torch.float16)
        Qd, Dd = Q.to(dev), Dh.to(dev)
        cfg = {"workload": f"single-query flash_maxsim Q[{Lq},{d}] x D[{B},{Ld},{d}] fp16", "B": B, "Lq": Lq,
               "Ld": Ld, "d": d}
        step = lambda: fm.flash_maxsim(Qd, Dd)  # noqa: E731
        algo_bytes = B * Ld * d * 2 + Lq * d * 2 + B * 4
        roof = {"bound": "hbm", "amount": algo_bytes, "unit": "GB/s", "kernel": "stream_fwd_kernel"}
        Qn, Dn = Q.float().numpy(), Dh.float().numpy()
        oracle_fn = lambda: oracle.maxsim(Qn, Dn)  # noqa: E731
        return cfg, step, B, roof, oracle_fn, B, "docs/s"
    if name == "c1_topk":
        # Config 1 scoring followed by top-100 selection (fused retrieval call).
        B, Lq, Ld, d, k = 5000, 32, 300, 128, 100
        Q = sim((Lq, d), 11, torch.float16)
        Dh = sim((B, Ld, d), 12, torch.float16)
        Qd, Dd = Q.to(dev), Dh.to(dev)
        cfg = {"workload": f"flash_maxsim_topk k={k}: Q[{Lq},{d}] x D[{B},{Ld},{d}] fp16", "B": B, "Lq": Lq,
               "Ld": Ld, "d": d, "k": k}
        step = lambda: fm.flash_maxsim_topk(Qd, Dd, k)  # noqa: E731
        algo_bytes = B * Ld * d * 2 + Lq * d * 2 + B * 4 * 2 + k * 12
        roof = {"bound": "hbm", "amount": algo_bytes, "unit": "GB/s", "kernel": "stream_fwd_kernel + topk"}
        Qn, Dn = Q.float().numpy(), Dh.float().numpy()

        def oracle_fn():
            oracle.topk(oracle.maxsim(Qn, Dn)[0], k)

        return cfg, step, B, roof, oracle_fn, B, "docs/s"
    if name == "c2":
        B, Lq, Ld, d = 1000, 1024, 1024, 128
        Q = sim((Lq, d), 21, torch.float16)
        Dh = sim((B, Ld, d), 22, torch.float16)
        Qd, Dd = Q.to(dev), Dh.to(dev)
        cfg = {"workload": f"single-query flash_maxsim Q[{Lq},{d}] x D[{B},{Ld},{d}] fp16", "B": B, "Lq": Lq,
               "Ld": Ld, "d": d}
        step = lambda: fm.flash_maxsim(Qd, Dd)  # noqa: E731
        roof = {"bound": "mfma", "amount": 2 * Lq * Ld * d * B, "unit": "TFLOP/s", "kernel": "tiled_fwd_kernel"}
        Qn, Dn = Q.float().numpy(), Dh[:8].float().numpy()
        oracle_fn = lambda: oracle.maxsim(Qn, Dn)  # noqa: E731
        return cfg, step, B, roof, oracle_fn, 8, "docs/s"
    if name == "c3":
        Nq, B, Lq, Ld, d = 100, 5000, 32, 300, 128
        Q = sim((Nq, Lq, d), 31, torch.float16)
        Dh = sim((B, Ld, d), 32, torch.float16)
        Qd, Dd = Q.to(dev), Dh.to(dev)
        cfg = {"workload": f"batched flash_maxsim Q[{Nq},{Lq},{d}] x D[{B},{Ld},{d}] fp16 shared docs",
               "Nq": Nq, "B": B, "Lq": Lq, "Ld": Ld, "d": d}
        step = lambda: fm.flash_maxsim_batched(Qd, Dd)  # noqa: E731
        roof = {"bound": "mfma", "amount": 2 * Nq * Lq * Ld * d * B, "unit": "TFLOP/s",
                "kernel": "tiled_fwd_kernel"}
        Qn, Dn = Q.float().numpy(), Dh[:50].float().numpy()
        oracle_fn = lambda: oracle.maxsim(Qn, Dn)  # noqa: E731
        return cfg, step, Nq * B, roof, oracle_fn, Nq * 50, "pairs/s"
    if name == "c4":
        B, Lq, Ld, d = 5000, 32, 1024, 128
        Q = sim((Lq, d), 41, torch.float16)
        codes = torch.empty(B, Ld, d, dtype=torch.uint8)
        scales = torch.empty(B, Ld, 1, dtype=torch.float16)
        mins = torch.empty(B, Ld, 1, dtype=torch.float16)
        for b0 in range(0, B, 500):  # bounded host memory
            Dc = sim((500, Ld, d), 42 + b0, torch.float32)
            c, s, m = fm.quantize_int8(Dc)
            codes[b0:b0 + 500], scales[b0:b0 + 500], mins[b0:b0 + 500] = c, s, m
        lengths = torch.randint(32, 1025, (B,), generator=torch.Generator().manual_seed(43), dtype=torch.int32)
        Qd, cd, sd, md, ld = (t.to(dev) for t in (Q, codes, scales, mins, lengths))
        tot = int(lengths.sum())
        cfg = {"workload": f"int8 fused-dequant varlen flash_maxsim_int8 Q[{Lq},{d}] x D[{B},{Ld},{d}] u8, "
                           f"len U[32,1024]", "B": B, "Lq": Lq, "Ld": Ld, "d": d, "sum_len": tot}
        step = lambda: fm.flash_maxsim_int8(Qd, cd, sd, md, ld)  # noqa: E731
        algo_bytes = tot * (d + 4) + Lq * d * 2 + B * 8
        roof = {"bound": "hbm", "amount": algo_bytes, "unit": "GB/s", "kernel": "stream_fwd_kernel"}
        Qn, cn = Q.float().numpy(), codes[:200].numpy()
        sn, mn, ln = scales[:200].float().numpy(), mins[:200].float().numpy(), lengths[:200].numpy()
        oracle_fn = lambda: oracle.maxsim_int8(Qn, cn, sn, mn, ln)  # noqa: E731
        return cfg, step, B, roof, oracle_fn, 200, "docs/s"
    if name == "c4_packed":
        # Config 4's docs (same seeds) quantised straight into the packed layout.
        B, Lq, Ld, d = 5000, 32, 1024, 128
        Q = sim((Lq, d), 41, torch.float16)
        lengths = torch.randint(32, 1025, (B,), generator=torch.Generator().manual_seed(43), dtype=torch.int32)
        Dg = torch.empty(B, Ld, d, dtype=torch.float32, device=dev)
        for b0 in range(0, B, 500):
            Dg[b0:b0 + 500] = sim((500, Ld, d), 42 + b0, torch.float32).to(dev)
        packed = fm.quantize_int8_packed(Dg, lengths)
        del Dg
        Qd = Q.to(dev)
        tot = int(lengths.sum())
        cfg = {"workload": f"int8 packed varlen flash_maxsim_int8_packed Q[{Lq},{d}] x {B} docs of U[32,1024] "
                           f"tokens, d={d} u8 ({packed.codes.shape[0]} packed rows)", "B": B, "Lq": Lq, "d": d,
               "sum_len": tot}
        step = lambda: fm.flash_maxsim_int8_packed(Qd, packed)  # noqa: E731
        algo_bytes = tot * (d + 4) + Lq * d * 2 + B * 16  # + tok_group, lengths, scores
        roof = {"bound": "hbm", "amount": algo_bytes, "unit": "GB/s", "kernel": "stream_fwd_kernel"}
        pc = packed.codes.cpu().numpy()
        tg, ln = packed.tok_group.cpu().numpy(), lengths.numpy()
        ps, pm = packed.scales.float().cpu().numpy(), packed.mins.float().cpu().numpy()
        nb = 200
        Lmax = int(ln[:nb].max())
        cn = np.zeros((nb, Lmax, d), np.uint8)
        sn = np.zeros((nb, Lmax), np.float32)
        mn = np.zeros((nb, Lmax), np.float32)
        for b in range(nb):  # padded copies of the first docs for the CPU oracle
            r0 = 4 * tg[b]
            cn[b, :ln[b]], sn[b, :ln[b]], mn[b, :ln[b]] = pc[r0:r0 + ln[b]], ps[r0:r0 + ln[b]], pm[r0:r0 + ln[b]]
        Qn, lnb = Q.float().numpy(), ln[:nb]
        oracle_fn = lambda: oracle.maxsim_int8(Qn, cn, sn, mn, lnb)  # noqa: E731
        return cfg, step, B, roof, oracle_fn, nb, "docs/s"
    if name == "quant":
        # quantize_int8 of config 4's docs on the GPU (HIP encoder), fp16 source.
        B, Ld, d = 5000, 1024, 128
        Dg = torch.empty(B, Ld, d, dtype=torch.float16, device=dev)
        for b0 in range(0, B, 500):
            Dg[b0:b0 + 500] = sim((500, Ld, d), 42 + b0, torch.float16).to(dev)
        cfg = {"workload": f"quantize_int8 of D[{B},{Ld},{d}] fp16 -> u8 codes + fp16 scales/mins", "B": B,
               "Ld": Ld, "d": d}
        step = lambda: fm.quantize_int8(Dg)  # noqa: E731
        algo_bytes = B * Ld * (d * 2 + d + 4)
        roof = {"bound": "hbm", "amount": algo_bytes, "unit": "GB/s", "kernel": "quantize_kernel"}
        Dn = Dg[:20].float().cpu().numpy()
        oracle_fn = lambda: oracle.quantize_int8(Dn)  # noqa: E731
        return cfg, step, B, roof, oracle_fn, 20, "docs/s"
    if name == "c5":
        B, Lq, Ld, d = 1000, 128, 512, 1024
        Q = sim((Lq, d), 51, torch.float16)
        Dh = sim((B, Ld, d), 52, torch.float16)
        Qd = Q.to(dev).requires_grad_(True)
        Dd = Dh.to(dev).requires_grad_(True)

        def step():
            s = fm.flash_maxsim_train(Qd, Dd)
            s.sum().backward()
            Qd.grad = None
            Dd.grad = None

        cfg = {"workload": f"train fwd+bwd flash_maxsim_train Q[{Lq},{d}] x D[{B},{Ld},{d}] fp16", "B": B,
               "Lq": Lq, "Ld": Ld, "d": d}
        # D read by the forward + dD written + the B*Lq rows of D gathered for dQ
        # + argmax written and read back (Q, dQ and scores are < 1 MB).
        algo_bytes = 2 * B * Ld * d * 2 + B * Lq * d * 2 + B * Lq * 4 * 2
        roof = {"bound": "hbm", "amount": algo_bytes, "unit": "GB/s", "kernel": "splitd_fwd_kernel + bwd kernels (whole step)"}
        Qn, Dn = Q.float().numpy(), Dh[:4].float().numpy()

        def oracle_fn():
            s, am, _ = oracle.maxsim(Qn, Dn, want_argmax=True)
            oracle.bwd(Qn, Dn, am, np.ones(4))

        return cfg, step, B, roof, oracle_fn, 4, "docs/s"
    if name == "copy":
        # Calibration for HBM byte counters: a plain device copy of the metric's D size.
        n = 5000 * 300 * 128
        src = torch.empty(n, dtype=torch.float16, device=dev).normal_()
        dst = torch.empty_like(src)
        cfg = {"workload": f"device copy of {n * 2} bytes (counter calibration)", "bytes": n * 2}
        step = lambda: dst.copy_(src)  # noqa: E731
        roof = {"bound": "hbm", "amount": 2 * n * 2, "unit": "GB/s", "kernel": "copy"}
        return cfg, step, 1, roof, (lambda: None), 1, "copies/s"
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
    ap.add_argument("--config", default="c1",
                    help="c1 (metric), c1_1000, c1_topk, c2, c3, c4, c4_packed, quant, c5, copy")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: every GPU box of this build has one MI355X, and the "
              "multi-GPU path (docs sharded across GPUs) is described in DESIGN.md, not run.", file=sys.stderr)
        raise SystemExit(2)

    import numpy as np
    import torch

    import oracle

    torch.cuda.set_device(0)
    cfg, step, units, roof, oracle_fn, oracle_units, unit = make_workload(args.config)
    for _ in range(args.warmup):
        step()
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
    for _ in range(args.steps):
        step()
    ev_end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1000.0 / args.steps
    kern_ms = ev_start.elapsed_time(ev_end) / args.steps  # average launch duration on the kernel's stream
    value = units / (ms_per_step / 1000.0)

    achieved = roof["amount"] / (kern_ms / 1000.0)
    if roof["unit"] == "GB/s":
        achieved /= 1e9
        peak = HBM_PEAK_GBS
    else:
        achieved /= 1e12
        peak = MFMA_F16_PEAK_TFLOPS
    traffic, traffic_src = measured_traffic(args.config)
    roofline = {"bound": roof["bound"], "achieved": round(achieved, 2), "peak": peak, "unit": roof["unit"],
                "frac": round(achieved / peak, 4), "traffic": traffic, "traffic_source": traffic_src,
                "algorithmic": roof["amount"], "kernel": roof["kernel"],
                "kernel_ms": round(kern_ms, 5)}

    cpu = None
    if not args.no_cpu and args.config != "copy":
        # Bounded sample: the oracle over `oracle_units` items of the same
        # workload, repeated until at least CPU_SAMPLE_S seconds have run.
        threads = oracle.default_threads()
        oracle_fn()  # warm
        calls = 0
        t = time.perf_counter()
        while True:
            oracle_fn()
            calls += 1
            el = time.perf_counter() - t
            if el >= CPU_SAMPLE_S and calls >= 3:
                break
        cpu = {"value": round(oracle_units * calls / el, 2), "unit": unit, "cores": threads, "kind": "port",
               "sample": f"{calls} x {oracle_units} {unit.split('/')[0]} of the same workload "
                         f"({el:.1f} s), float64 oracle (oracle/maxsim_oracle.c) on {threads} threads, "
                         f"{cpu_model()}"}

    line = {
        "metric": METRIC if args.config == "c1" else f"{args.config}: {cfg['workload']}",
        "value": round(value, 1),
        "unit": unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": cfg,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
