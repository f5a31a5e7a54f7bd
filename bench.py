"""Throughput of the TCQ Viterbi quantizer on one MI355X: the C3 headline workload.

Workload (metric format TCQ275X2 = K=3 D4, 8 subsets, h=2): W [4096, 14336] bf16
Student-t(5) * 0.02 with 143 outlier columns * 20, H = X^T X / 2048 from X [2048, 14336] N(0, 1), damping
0.2 * mean(diag H_rot). The weight matrix is rotated (suh, FWHT-256), given its row scale (fp16 d_row +
5-bit e per (row, 256-block)), and H is factored (U, diag_w) before the timed region, as inputs of the path.

One step quantizes the whole matrix the way src/liqk_v2.py:957-980 drives it: for each 256-column block and
each 16-column sub-block, one two-pass tail-biting Viterbi over the 256 tiles of 16 rows x 16 columns
(src/liqk_v2.py:917-919 -> src/tcq_proto.py:584-609), returning codes for PACK. All inputs are resident
in HBM when the timed region starts.

Prints one JSON line (driver contract). `roofline` is the dominant kernel (the Viterbi) against the gfx950
fp32 VALU peak, from HIP events recorded around every Viterbi pass inside the timed region on the stream
the kernels run on; `cpu_baseline` is the C oracle (a scalar-per-thread port of the reference semantics,
OpenMP over tiles) timed on this host on a bounded sample of the same workload.
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
sys.path.insert(0, str(ROOT / "ltq-research_amd"))

M_ROWS, K_COLS, N_OUTLIER, N_ACT = 4096, 14336, 143, 2048
FORMAT = "TCQ275X2"
TB_WINDOW = 32          # TCQ_TB_WIN default (src/liqk_v2.py:918)
DAMP = 0.2              # 0.02 * TCQ_DAMP_MULT (src/liqk_v2.py:1061-1063)
# gfx950 VALU: one non-packed wave64 instruction per 4 cycles per SIMD (measured: 3.1-3.5e13 lane-ops/s for
# v_sub_f32 / v_alignbit_b32 at 1-4 waves per SIMD) = 256 CU x 4 SIMD x 16 lanes x 2.4 GHz
VALU_PEAK_TOPS = 39.3
LANE_OPS_PER_STEP = {0: 2.0, 1: 4.5, 2: 8.25, 3: 8.25}  # per state, per weight, per gain slot (radix-4 ACS)


def student_t(shape, gen, dev):
    """Student-t(5) = z / sqrt(chi2_5 / 5) with chi2_5 from 5 squared normals (seedable)."""
    import torch
    z = torch.randn(shape, generator=gen, device=dev)
    chi2 = torch.zeros(shape, device=dev)
    for _ in range(5):
        chi2 += torch.randn(shape, generator=gen, device=dev).square()
    return z / (chi2 / 5).sqrt()


def prepare(dev, rows=M_ROWS, cols=K_COLS):
    """Inputs of the quantizer on the device: Viterbi tiles [nblk, 16, rows/16, 256] (x / d per row block,
    tile-major), per-position weights [nblk, 16, 256] (diag_w of the sub-block repeated over 16 rows)."""
    import torch
    from ltq_amd.formats import TCQ_CONFIG
    from ltq_amd import rotation

    # seeded device generators (W: 0, activations: 1, outlier columns: 2 on the CPU)
    W = student_t((rows, cols), torch.Generator(device=dev).manual_seed(0), dev) * 0.02
    cols_out = torch.randperm(cols, generator=torch.Generator().manual_seed(2))[:max(1, cols * N_OUTLIER // K_COLS)]
    W[:, cols_out.to(dev)] *= 20
    W = W.to(torch.bfloat16)
    X = torch.randn((N_ACT, cols), generator=torch.Generator(device=dev).manual_seed(1), device=dev)
    H = (X.T @ X) / N_ACT
    del X
    W_rot, H_rot, suh = rotation.compute_optimal_suh(W, H, seed=1337)
    del H
    H_rot.diagonal().add_(DAMP * H_rot.diagonal().mean().clamp(min=1e-8))
    L_flip = torch.linalg.cholesky(H_rot.flip(0, 1))
    del H_rot
    U = torch.linalg.solve_triangular(L_flip, torch.eye(cols, device=dev), upper=False).flip(0, 1)
    del L_flip
    diag_w = 1.0 / (torch.diagonal(U) ** 2).clamp(min=1e-12)
    del U
    cfg = TCQ_CONFIG[FORMAT]
    nblk = cols // 256
    # row scale (src/liqk_v2.py:938-946)
    rms_rb = W_rot.view(rows, nblk, 256).square().mean(dim=2).sqrt().clamp(min=1e-10) * cfg.get("scale", 1.0)
    d_row = torch.exp(torch.log(rms_rb).mean(dim=1)).to(torch.float16).to(torch.float32).clamp(min=1e-8)
    e_rb = torch.round(torch.log2(rms_rb / d_row.unsqueeze(1)) / 0.25).clamp(-16, 15)
    d_rb = (d_row.unsqueeze(1) * torch.exp2(0.25 * e_rb)).clamp(min=1e-8)
    xs = W_rot.view(rows, nblk, 16, 16) / d_rb.view(rows, nblk, 1, 1)
    # tile n of sub-block (b, s) = rows 16n..16n+15, columns 16s..16s+15 of block b, row-major in the tile
    tiles = xs.view(rows // 16, 16, nblk, 16, 16).permute(2, 3, 0, 1, 4).contiguous().view(nblk, 16, rows // 16, 256)
    wts = diag_w.view(nblk, 16, 16).repeat(1, 1, 16).contiguous()
    return tiles, wts


def lane_ops_per_launch(cfg, tiles, steps):
    G = cfg.get("n_cand", 0) or (1 << cfg["h"])
    return tiles * steps * LANE_OPS_PER_STEP[int(cfg.get("pp", 0))] * 1024 * G


def read_traffic():
    """HBM bytes per Viterbi launch measured with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE (committed summary)."""
    p = ROOT / "profiles" / "tcq_viterbi_c3_tcq275x2_traffic.txt"
    if not p.exists():
        return None
    for line in p.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch"):
            return float(line.split("=")[1])
    return None


def cpu_baseline(tiles, wts, budget_s):
    """The C oracle (OpenMP over tiles) on the first sub-blocks, in quantization order, until budget_s is spent."""
    import numpy as np
    from oracle import ref
    from ltq_amd.formats import make_format, TCQ_CONFIG
    f = make_format(FORMAT)
    cfg = TCQ_CONFIG[FORMAT]
    cores = min(16, len(os.sched_getaffinity(0)))
    ref.lib()
    done, t0 = 0, time.perf_counter()
    nsub = 0
    for b, s in ((b, s) for b in range(tiles.shape[0]) for s in range(tiles.shape[1])):
        x = tiles[b, s].cpu().numpy()
        w = wts[b, s].cpu().numpy()
        ref.viterbi_ub_cuda_ref(x, f.lut, f.K, 10, 359, f.gain_tab, sub=f.sub, wts=w, n_cand=cfg.get("n_cand", 0),
                                tail_biting=True, tb_window=TB_WINDOW, m_extra=f.masks[1:], pair_parity=int(cfg["pp"]),
                                return_code=True, nthreads=cores)
        done += x.size
        nsub += 1
        if time.perf_counter() - t0 > budget_s:
            break
    dt = time.perf_counter() - t0
    return {"value": round(done / dt / 1e6, 4), "unit": "Mweights/s", "cores": cores, "kind": "port",
            "sample": f"oracle/ltq_oracle.c two-pass tail-biting Viterbi of the first {nsub} sub-block(s) in order "
                      f"({nsub} x {tiles.shape[2]} tiles x 256 weights = {done} weights) in {dt:.1f} s on {cores} threads"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU baseline sample (0 = skip)")
    ap.add_argument("--blocks", type=int, default=0, help="column blocks per step (0 = all 56; profiling runs only)")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="profiling runs: first copy this many MiB device-to-device (a known-size kernel that "
                         "calibrates the FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the Viterbi path is row-sharded with no exchange on the hot path, "
              "and this build runs and reports a single MI355X (--gpus 1).", file=sys.stderr)
        sys.exit(2)

    import torch
    from ltq_amd import tcq_proto
    from ltq_amd.formats import TCQ_CONFIG, make_format

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cfg = TCQ_CONFIG[FORMAT]
    f = make_format(FORMAT)
    if args.copy_mib:
        a = torch.ones(args.copy_mib << 18, device=dev)
        torch.empty_like(a).copy_(a)
        torch.cuda.synchronize()
        del a
    tiles, wts = prepare(dev)
    nblk = args.blocks or tiles.shape[0]
    lut = torch.tensor(f.lut, device=dev)
    gains = torch.tensor(f.gain_tab, device=dev)
    n_cand = cfg.get("n_cand", 0)
    kw = dict(sub=f.sub, n_cand=n_cand, m_extra=f.masks[1:], pair_parity=int(cfg["pp"]))
    h = 128
    stream = torch.cuda.current_stream()

    def step(events=None):
        codes = []
        for b in range(nblk):
            for s in range(16):
                x, w = tiles[b, s], wts[b, s]
                # pass 1: window [h - 32, h + 32) for the middle state; pass 2: closed path from it
                # (the two passes of src/tcq_proto.py:584-609, issued individually to time each launch)
                if events is not None:
                    e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
                    e[0].record(stream)
                _, mid = tcq_proto.viterbi_ub_cuda(x, lut, f.K, 10, 359, gains, wts=w.view(1, 256).expand(x.shape[0], 256),
                                                   _mid=TB_WINDOW, _steps=2 * TB_WINDOW, _rot=h - TB_WINDOW, **kw)
                if events is not None:
                    e[1].record(stream)
                out = tcq_proto.viterbi_ub_cuda(x, lut, f.K, 10, 359, gains, wts=w.view(1, 256).expand(x.shape[0], 256),
                                                init_state=mid, return_code=True, _tail=True, _rot=h, **kw)
                if events is not None:
                    e[2].record(stream)
                    events.append(e)
                codes.append(out[2])
        return codes

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    events = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(events)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms_step = dt / args.steps * 1e3
    weights = nblk * 16 * tiles.shape[2] * 256
    value = weights / (dt / args.steps) / 1e6

    t_p1 = sum(e[0].elapsed_time(e[1]) for e in events) / len(events) * 1e-3
    t_p2 = sum(e[1].elapsed_time(e[2]) for e in events) / len(events) * 1e-3
    ntile = tiles.shape[2]
    ops = (lane_ops_per_launch(cfg, ntile, 2 * TB_WINDOW) + lane_ops_per_launch(cfg, ntile, 256)) / 2
    avg = (t_p1 + t_p2) / 2
    achieved = ops / avg / 1e12
    traffic = read_traffic()
    out = {
        "metric": "Mweights/s quantized (K=3 D4, 4096x14336) on 1 GPU; % VALU ACS roofline",
        "value": round(value, 3), "unit": "Mweights/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_step, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic, generated on the device (Student-t(5)*0.02 bf16 weights, 143 outlier "
                                "columns x20; H from 2048 N(0,1) rows; seeds 0/1/2)",
        "config": {"workload": f"C3 down_proj {M_ROWS}x{K_COLS} {FORMAT} (K=3 D4, nl=8, h=2) tail-biting "
                               f"tb_window={TB_WINDOW}, Viterbi of all {nblk * 16} sub-blocks per step "
                               f"({ntile} tiles per launch, 2 passes)",
                   "stages_timed": ["viterbi_tail_biting"], "format": FORMAT, "rows": M_ROWS,
                   "cols": nblk * 256, "parallelism": "single GPU"},
        "roofline": {"bound": "valu", "achieved": round(achieved, 3), "peak": VALU_PEAK_TOPS,
                     "unit": "TFLOP/s (fp32 VALU lane-ops/s x 1e-12)", "frac": round(achieved / VALU_PEAK_TOPS, 4),
                     "traffic": traffic, "kernel": "tcq_viterbi_kernel<10,2,8,4>",
                     "avg_launch_us": round(avg * 1e6, 2), "pass1_us": round(t_p1 * 1e6, 2),
                     "pass2_us": round(t_p2 * 1e6, 2), "lane_ops_per_launch": ops},
    }
    if args.cpu_seconds > 0:
        out["cpu_baseline"] = cpu_baseline(tiles, wts, args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
