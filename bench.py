"""Throughput of the TCQ Viterbi quantizer on one MI355X: the C3 headline workload.

Workload (metric format TCQ275X2 = K=3 D4, 8 subsets, h=2): W [4096, 14336] bf16
Student-t(5) * 0.02 with 143 outlier columns * 20, H = X^T X / 2048 from X [2048, 14336] N(0, 1) activations in
bf16 (accumulated by ltq_cov_accumulate, the reference's _CovAccumulator, before the timed region and reported
separately under `h_build`), damping 0.2 * mean(diag H_rot). W and H are resident in HBM when the timed region
starts.

One step is quantize_matrix_liqk_v2 with PACK plus .ltq slice packing: rotation (suh, FWHT-256), factors of
H_rot, row scale, and for each 256-column block and each 16-column sub-block one two-pass tail-biting Viterbi
over the 256 tiles of 16 rows x 16 columns (src/liqk_v2.py:917-919 -> src/tcq_proto.py:584-609) with the LDLQ
feedback, then the c_row / suh refit.

Prints one JSON line (driver contract). `roofline` is the dominant kernel (the Viterbi) against the gfx950
fp32 VALU peak, from HIP events carried by both Viterbi launches of one sub-block in 17 inside the timed
region (17 is prime to the 16 sub-blocks of a column block, so every sub-block position is sampled alike); `cpu_baseline` is the reference's CPU path -- torch, eager, every core
of this host (oracle/torch_viterbi.py restates viterbi_ub with the production semantics, pinned to the
reference's outputs) plus the LDLQ feedback -- on the first sub-blocks of the same matrix, extrapolated to the
whole matrix; `cpu_baseline_c_port` is the C oracle on the same tiles (Viterbi stage only).
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
    """W [rows, cols] bf16 and H [cols, cols] fp32 on the device (seeded device generators: W 0, activations 1;
    outlier columns: seed 2 on the CPU)."""
    import torch
    W = student_t((rows, cols), torch.Generator(device=dev).manual_seed(0), dev) * 0.02
    cols_out = torch.randperm(cols, generator=torch.Generator().manual_seed(2))[:max(1, cols * N_OUTLIER // K_COLS)]
    W[:, cols_out.to(dev)] *= 20
    W = W.to(torch.bfloat16)
    X = torch.randn((N_ACT, cols), generator=torch.Generator(device=dev).manual_seed(1), device=dev)
    H, h_build = build_hessian(X.to(torch.bfloat16))
    return W, H, h_build


def build_hessian(X):
    """H = X^T X / n through CovAccumulator (one ltq_cov_accumulate + ltq_cov_finalize), timed with HIP events after
    one untimed warm-up accumulation: the H-build figures reported beside the step."""
    import torch
    from ltq_amd.hessian import CovAccumulator
    CovAccumulator().add(X)
    stream = torch.cuda.current_stream()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    acc = CovAccumulator()
    ev[0].record(stream)
    acc.add(X)
    ev[1].record(stream)
    H = acc.get()
    ev[2].record(stream)
    torch.cuda.synchronize()
    n, K = X.shape
    nt = (K + 127) // 128
    flop = 2.0 * n * 128 * 128 * nt * (nt + 1) // 2  # the lower-triangle 128 x 128 tiles the kernel computes
    t_acc = ev[0].elapsed_time(ev[1]) * 1e-3
    return H, {"rows": n, "cols": K, "dtype": "bf16", "accumulate_ms": round(t_acc * 1e3, 4),
               "finalize_ms": round(ev[1].elapsed_time(ev[2]), 4), "mfma_tflops": round(flop / t_acc / 1e12, 1),
               "frac_bf16_dense_peak": round(flop / t_acc / 2.5e15, 4),
               "kernel": "ltq_cov_accumulate (cov_kernel<bf16>), fp32 MFMA accumulation into fp64 H"}


def block_inputs(W, H):
    """W_rot, U, U_blks_inv[0], diag_w and the block scales of the first 256-column block, computed by the product
    path (rotation, factors, row scale) and copied to the host: the inputs of the CPU baselines."""
    from ltq_amd import liqk, rotation
    from ltq_amd.formats import TCQ_CONFIG
    cfg = TCQ_CONFIG[FORMAT]
    W_rot, H_rot, _ = rotation.compute_optimal_suh(W.float(), H.float(), seed=1337)
    U, diag_w, Ub_inv = liqk.factor_hessian(H_rot, DAMP)
    _, _, d = liqk.row_scale(W_rot, cfg)
    return (W_rot[:, :256].cpu(), U[:256, :256].cpu(), Ub_inv[0].cpu(), diag_w[:256].cpu(), d[:, 0].cpu())


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline_torch(inputs, budget_s, total_subblocks):
    """The CPU baseline the benchmark plan specifies: the reference's CPU path -- torch on the host, eager, every
    available core -- over the first 256-column block of the same matrix with its LDLQ feedback (src/liqk_v2.py:948-970: torch
    matmuls), the Viterbi by oracle/torch_viterbi.py (the torch restatement of viterbi_ub with the kernel's D4 /
    tail-biting semantics). Sub-blocks run in order until budget_s is spent (at least one); the whole-matrix rate
    is extrapolated from them."""
    import numpy as np
    import torch
    from oracle import torch_viterbi
    from ltq_amd.formats import TCQ_CONFIG, make_format
    cfg, f = TCQ_CONFIG[FORMAT], make_format(FORMAT)
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    W_rot, U_blk, U_inv, diag_w, d = (t.float() for t in inputs)
    rows = W_rot.shape[0]
    w_sub = W_rot.clone()
    inv_d = 1.0 / d.clamp(min=1e-8).unsqueeze(1)
    done, t0 = 0, time.perf_counter()
    for ib in range(16):
        s0, s1 = 16 * ib, 16 * ib + 16
        x = (w_sub[:, s0:s1] * inv_d).contiguous().view(rows // 16, 256).numpy()
        rec, _, _ = torch_viterbi.viterbi_ub_cuda_torch(x, f.lut, f.K, 10, 359, f.gain_tab, sub=16,
                                                        wts=np.tile(diag_w[s0:s1].numpy(), 16),
                                                        n_cand=cfg.get("n_cand", 0), tail_biting=True,
                                                        tb_window=TB_WINDOW, m_extra=f.masks[1:],
                                                        pair_parity=int(cfg["pp"]))
        g_sub = torch.from_numpy(rec).view(rows, 16)
        if s1 < 256:
            err = (w_sub[:, s0:s1] - d.unsqueeze(1) * g_sub) @ U_inv[s0:s1, s0:s1]
            w_sub[:, s1:] -= err @ U_blk[s0:s1, s1:]
        done += 1
        if time.perf_counter() - t0 > budget_s:
            break
    dt = time.perf_counter() - t0
    per_sub = dt / done
    total = per_sub * total_subblocks
    weights = rows * 16 * total_subblocks
    return {"value": round(weights / total / 1e6, 5), "unit": "Mweights/s", "cores": cores, "kind": "port",
            "extrapolated": True, "cpu_model": cpu_model(), "os_cpu_count": os.cpu_count(),
            "sample": f"torch (eager, {cores} threads) restatement of the reference's CPU Viterbi "
                      f"(oracle/torch_viterbi.py, src/tcq_proto.py:327-419 with the kernel's D4 / tail-biting "
                      f"semantics) plus the LDLQ sub-block feedback in torch, over the first {done} sub-blocks of "
                      f"the first 256-column block ({rows} x {16 * done} weights) in {dt:.1f} s; whole matrix "
                      f"extrapolated x{total_subblocks / done:.0f} ({per_sub:.2f} s per sub-block)"}


def cpu_baseline_port(inputs, budget_s):
    """The C oracle (oracle/ltq_oracle.c, OpenMP over tiles) on the same sub-blocks: Viterbi stage only."""
    import numpy as np
    from oracle import ref
    from ltq_amd.formats import TCQ_CONFIG, make_format
    f = make_format(FORMAT)
    cfg = TCQ_CONFIG[FORMAT]
    W_rot, _, _, diag_w, d = inputs
    rows = W_rot.shape[0]
    cores = min(16, len(os.sched_getaffinity(0)))
    ref.lib()
    xs = (W_rot.float() / d.clamp(min=1e-8).unsqueeze(1)).view(rows // 16, 16, 16, 16).permute(2, 0, 1, 3)
    xs = xs.contiguous().view(16, rows // 16, 256)
    done, nsub, t0 = 0, 0, time.perf_counter()
    while time.perf_counter() - t0 <= budget_s:
        s = nsub % 16
        ref.viterbi_ub_cuda_ref(xs[s].numpy(), f.lut, f.K, 10, 359, f.gain_tab, sub=f.sub,
                                wts=np.tile(diag_w[16 * s:16 * s + 16].numpy(), 16), n_cand=cfg.get("n_cand", 0),
                                tail_biting=True, tb_window=TB_WINDOW, m_extra=f.masks[1:],
                                pair_parity=int(cfg["pp"]), return_code=True, nthreads=cores)
        done += xs.shape[1] * 256
        nsub += 1
    dt = time.perf_counter() - t0
    return {"value": round(done / dt / 1e6, 4), "unit": "Mweights/s", "cores": cores, "kind": "port",
            "sample": f"oracle/ltq_oracle.c two-pass tail-biting Viterbi (a C port, OpenMP over tiles), {nsub} "
                      f"sub-block launches over the first block's sub-blocks ({done} weights) in {dt:.1f} s on "
                      f"{cores} threads; the Viterbi stage only, to compare with breakdown.mweights_s_viterbi"}


def lane_ops_per_launch(cfg, tiles, steps):
    G = cfg.get("n_cand", 0) or (1 << cfg["h"])
    return tiles * steps * LANE_OPS_PER_STEP[int(cfg.get("pp", 0))] * 1024 * G


def viterbi_event_totals(records):
    """(seconds, lane-ops, launches) summed over tcq_proto timing-hook records: each record is one Viterbi call
    (both passes of a tail-biting call) with one event pair per kernel launch (each launch's own start / end) and
    the (steps, gain slots) of every pass."""
    secs = ops = 0.0
    n = 0
    for r in records:
        secs += sum(e0.elapsed_time(e1) for e0, e1 in r["ev"]) * 1e-3
        for steps, G in r["launches"]:
            ops += r["tiles"] * steps * LANE_OPS_PER_STEP[r["pp"]] * 1024 * G
            n += 1
    return secs, ops, n


def read_traffic():
    """HBM bytes per Viterbi launch measured with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE (committed summary)."""
    p = ROOT / "profiles" / "tcq_viterbi_c3_tcq275x2_traffic.txt"
    if not p.exists():
        return None
    for line in p.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch"):
            return float(line.split("=")[1])
    return None


HBM_PEAK_GBS = 8000.0      # MI355X HBM3E
MFMA_FP32_PEAK_TFLOPS = 157.3


class DeviceEvent:
    """A HIP timing event (hipEventCreateWithFlags, hipEventDisableSystemFence: an event only used to measure
    time). record(stream) enqueues it as a marker, as torch.cuda.Event does; `handle` (the hipEvent_t) lets
    tcq_proto hand it to the Viterbi launches themselves (ltq_viterbi_timing -> hipExtLaunchKernelGGL), which
    stamp it with the dispatch's own start / end time. A marker between two kernels costs about 5 us of idle
    dispatch gap on each side on MI355X (measured against the kernel trace), time the kernel does not spend.
    elapsed_time(end) in ms."""
    _hip = None

    @classmethod
    def _runtime(cls):
        if cls._hip is None:
            import ctypes
            import torch
            torch.cuda.init()
            path = next((ln.split()[-1] for ln in open("/proc/self/maps") if "libamdhip64.so" in ln), "libamdhip64.so")
            h = ctypes.CDLL(path)
            h.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
            h.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
            h.hipEventSynchronize.argtypes = [ctypes.c_void_p]
            h.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
            h.hipEventDestroy.argtypes = [ctypes.c_void_p]
            for f in ("hipEventCreateWithFlags", "hipEventRecord", "hipEventSynchronize", "hipEventElapsedTime",
                      "hipEventDestroy"):
                getattr(h, f).restype = ctypes.c_int
            cls._hip = h
        return cls._hip

    def __init__(self):
        import ctypes
        self._ev = ctypes.c_void_p()
        rc = self._runtime().hipEventCreateWithFlags(ctypes.byref(self._ev), 0x20000000)  # DisableSystemFence
        if rc != 0:
            raise RuntimeError(f"hipEventCreateWithFlags: HIP error {rc}")

    @property
    def handle(self):
        return self._ev.value

    def record(self, stream=None):
        import torch
        st = stream if stream is not None else torch.cuda.current_stream()
        rc = self._hip.hipEventRecord(self._ev, st.cuda_stream)
        if rc != 0:
            raise RuntimeError(f"hipEventRecord: HIP error {rc}")

    def elapsed_time(self, end):
        import ctypes
        ms = ctypes.c_float()
        if self._hip.hipEventSynchronize(end._ev) != 0 or self._hip.hipEventElapsedTime(ctypes.byref(ms), self._ev,
                                                                                         end._ev) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value

    def __del__(self):
        if self._ev and self._hip is not None:
            self._hip.hipEventDestroy(self._ev)
            self._ev = None


class KernelTimer:
    """Kernel times of selected product calls inside the timed steps. Each wrapped call launches one library
    kernel; the call arms ltq_kernel_timing with a start / stop DeviceEvent pair, so that launch carries the
    events (hipExtLaunchKernelGGL stamps them with the dispatch's own start and end: no marker packets around
    the kernel, no allocator or host work inside the interval). Each record is (name, start, end, algorithmic
    bytes, flops)."""

    def __init__(self):
        self.records = []
        self.active = False
        self._undo = []

    def _wrap(self, owner, attr, name_fn):
        from ltq_amd import _lib
        lib = _lib.lib()
        orig = getattr(owner, attr)

        def timed(*a, **k):
            if not self.active:
                return orig(*a, **k)
            e0, e1 = DeviceEvent(), DeviceEvent()
            lib.ltq_kernel_timing(e0.handle, e1.handle, 1)
            try:
                out = orig(*a, **k)
            finally:
                lib.ltq_kernel_timing(None, None, 0)
            name, nbytes, flops = name_fn(a, k, out)
            if name:
                self.records.append((name, e0, e1, nbytes, flops))
            return out

        setattr(owner, attr, timed)
        self._undo.append((owner, attr, orig))

    def install(self):
        from ltq_amd import _lib, liqk, ltq_file, rotation

        def rows_fn(a, k, out):
            x = a[0]
            n = x.numel()
            tag = "fwht_rows_W" if x.dtype != out.dtype else ("fwht_rows_H" if x.shape[0] == x.shape[1] else "")
            return tag, n * (x.element_size() + 4), 0

        def cols_fn(a, k, out):
            x = a[0]
            return ("fwht_cols_H" if x.shape[0] == x.shape[1] else ""), x.numel() * 8, 0

        def scale_fn(a, k, out):
            W = a[0]
            return "row_scale", W.numel() * 4 + W.shape[0] * (4 + 5 * (W.shape[1] // 256)), 0

        def pack_fn(a, k, out):
            idx = a[0]
            return "pack_slice", idx.numel() * 3 + out.numel(), 0

        self._wrap(rotation, "fwht_rows", rows_fn)
        self._wrap(rotation, "fwht_cols", cols_fn)
        self._wrap(liqk, "row_scale", scale_fn)
        self._wrap(ltq_file, "pack_slice_device", pack_fn)

        def upd_fn(a, k, out):
            M, N = a[6], a[7]
            return "ldlq_update", 8 * M * N + 4 * 256 * (N + M), 2.0 * M * 256 * N

        self._wrap(_lib.lib(), "ltq_ldlq_update", upd_fn)

    def uninstall(self):
        for owner, attr, orig in reversed(self._undo):
            setattr(owner, attr, orig)
        self._undo = []

    def summary(self, steps):
        """{name: {ms per step, GB/s, HBM fraction (and TFLOP/s, MFMA fraction)}} over the timed steps."""
        agg = {}
        for name, e0, e1, nbytes, flops in self.records:
            t = e0.elapsed_time(e1) * 1e-3
            a = agg.setdefault(name, [0.0, 0.0, 0.0, 0])
            a[0] += t
            a[1] += nbytes
            a[2] += flops
            a[3] += 1
        out = {}
        for name, (t, nb, fl, n) in agg.items():
            gbs = nb / t / 1e9
            d = {"calls_per_step": n // steps, "ms_per_step": round(t / steps * 1e3, 3),
                 "algorithmic_bytes_per_call": int(nb / n), "gb_s": round(gbs, 1),
                 "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
            if fl:
                d["tflop_s"] = round(fl / t / 1e12, 1)
                d["frac_mfma_fp32"] = round(fl / t / 1e12 / MFMA_FP32_PEAK_TFLOPS, 4)
            out[name] = d
        return out


C5_ROWS, C5_COLS = 262144, 2560  # K=4 D4 rings = TCQ375X; TCQ4X on request
RING_SCALES = 3  # quantize_rings' scale candidates (src/ple_quant.py:53)
# the reference's published ring-mode figure: TCQ4X:rot (3 scales x 2 passes), 2.82e9 values in 33.18 s = 84.9
# Mvalues/s (GPU unstated)
RING_PUBLISHED = {"TCQ4X": 84.9}


def prepare_rings(dev, rows):
    """C5 table [rows, 2560] bf16: N(0, 0.02^2) times a per-row log-normal(0, 0.5) norm (seeds 0 and 1)."""
    import torch
    W = torch.randn((rows, C5_COLS), generator=torch.Generator(device=dev).manual_seed(0), device=dev) * 0.02
    s = torch.exp(0.5 * torch.randn((rows, 1), generator=torch.Generator(device=dev).manual_seed(1), device=dev))
    return (W * s).to(torch.bfloat16)


def cpu_baseline_rings(W_sample, budget_s, fmt_name):
    """oracle/ple_ref.py (the ring quantizer over the C oracle Viterbi, OpenMP over rings) on a few rows, cycled
    until budget_s is spent."""
    from oracle import ple_ref, ref
    from ltq_amd.formats import TCQ_CONFIG, make_format
    ref.lib()
    cfg, fmt = TCQ_CONFIG[fmt_name], make_format(fmt_name)
    cores = min(16, len(os.sched_getaffinity(0)))
    done, k, t0 = 0, 0, time.perf_counter()
    while time.perf_counter() - t0 <= budget_s:
        row = W_sample[k % W_sample.shape[0]:k % W_sample.shape[0] + 1]
        ple_ref.quantize_rings_ref(row, cfg, fmt, rot=True)
        done += row.numel()
        k += 1
    dt = time.perf_counter() - t0
    return {"value": round(done / dt / 1e6, 5), "unit": "Mvalues/s", "cores": cores, "kind": "port",
            "sample": f"oracle/ple_ref.py quantize_rings_ref (3 scales, two-pass tail-biting Viterbi of the C oracle) "
                      f"on {k} rows of 2560 values ({done} values) cycling over {W_sample.shape[0]} rows of the table, "
                      f"{dt:.1f} s on up to {cores} OpenMP threads"}


def run_rings(args):
    """--workload c5: one step = quantize_rings_packed over the whole C5 table (ring rotation, 3 fp16 scales x
    two-pass tail-biting Viterbi per ring, selection, ring records)."""
    import torch
    from ltq_amd import ple_quant, tcq_proto
    from ltq_amd.formats import TCQ_CONFIG
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    rows = args.rows or C5_ROWS
    W = prepare_rings(dev, rows)
    fmt_name = args.format or "TCQ375X"
    step = lambda: ple_quant.quantize_rings_packed(W, fmt_name, rot=True)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    tcq_proto.LAUNCH_EVENTS, tcq_proto.LAUNCH_SAMPLE, tcq_proto._launch_count = [], 1, 0
    tcq_proto.EVENT_FACTORY = DeviceEvent
    t0 = time.perf_counter()
    for _ in range(args.steps):
        out = step()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    evs, tcq_proto.LAUNCH_EVENTS = tcq_proto.LAUNCH_EVENTS, None
    secs, ops, n_launch = viterbi_event_totals(evs)
    t_vit = secs / args.steps
    cfg = TCQ_CONFIG[fmt_name]
    nl = 4 << len(cfg.get("m_extra", ()))
    achieved = ops / secs / 1e12
    value = W.numel() / (dt / args.steps) / 1e6
    pub = RING_PUBLISHED.get(fmt_name)
    res = {
        "metric": f"Mvalues/s quantized rings ({fmt_name}, 3 scales x 2 passes, {rows}x{C5_COLS} row table) on 1 GPU; "
                  f"% VALU ACS roofline",
        "value": round(value, 3), "unit": "Mvalues/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(dt / args.steps * 1e3, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": round(value / pub, 3) if pub else None,
        "dtype": "f32",
        "data": "synthetic, generated on the device (N(0, 0.02^2) x per-row log-normal(0, 0.5) norm, bf16; seeds 0/1)",
        "config": {"workload": f"C5 row table {rows}x{C5_COLS} {fmt_name} rings: FWHT-256 per ring, 3 fp16 scales "
                               f"x two-pass tail-biting Viterbi (tb_window 0), selection, ring records",
                   "format": fmt_name, "rows": rows, "cols": C5_COLS, "parallelism": "single GPU"},
        "roofline": {"bound": "valu", "timed_on": "a HIP start / stop event pair carried by each Viterbi "
                                                  "launch of the timed steps (hipExtLaunchKernelGGL)",
                     "achieved": round(achieved, 3), "peak": VALU_PEAK_TOPS,
                     "unit": "TFLOP/s (fp32 VALU lane-ops/s x 1e-12)", "frac": round(achieved / VALU_PEAK_TOPS, 4),
                     "traffic": None, "kernel": f"tcq_viterbi_kernel<10,2,{int(cfg.get('pp', 0))},{nl},{8 if int(cfg.get('pp', 0)) == 0 else 1}>",
                     "viterbi_ms_per_step": round(t_vit * 1e3, 2),
                     "viterbi_launches_per_step": n_launch // args.steps},
        "breakdown": {"mvalues_s_viterbi": round(W.numel() / t_vit / 1e6, 3), "bits_per_value": out[1]},
    }
    if args.cpu_seconds > 0:
        res["cpu_baseline"] = cpu_baseline_rings(W[:64].float().cpu(), args.cpu_seconds, fmt_name)
    print(json.dumps(res), flush=True)


C4_EXPERTS, C4_HIDDEN, C4_INTER, C4_ACT_ROWS = 128, 2048, 768, 256
C4_FORMAT = "TCQ275Y3"  # K=3 D4, 16-subset labels, 3-bit gains over 4 candidates (closed-form table)


def prepare_experts(dev, n_exp):
    """C4: per expert the fused gate_up_proj [2 x 768, 2048] and down_proj [2048, 768], bf16 Student-t(5) x 0.02,
    and their Hessians from 256 N(0, 1) activation rows each (2048- and 768-dim), accumulated by
    ltq_cov_accumulate (seeds: weights 10 + e, activations 20000 + e). Returns (gate_up, H_in, down, H_mid,
    H-build milliseconds)."""
    import torch
    from ltq_amd.hessian import CovAccumulator
    gu, H_in, dn, H_mid = [], [], [], []
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t_h = 0.0
    for e in range(n_exp):
        g = torch.Generator(device=dev).manual_seed(10 + e)
        gu.append((student_t((2 * C4_INTER, C4_HIDDEN), g, dev) * 0.02).to(torch.bfloat16))
        dn.append((student_t((C4_HIDDEN, C4_INTER), g, dev) * 0.02).to(torch.bfloat16))
        ga = torch.Generator(device=dev).manual_seed(20000 + e)
        xs = [torch.randn((C4_ACT_ROWS, k), generator=ga, device=dev).to(torch.bfloat16) for k in (C4_HIDDEN, C4_INTER)]
        ev0.record()
        hs = []
        for x in xs:
            acc = CovAccumulator()
            acc.add(x)
            hs.append(acc.get())
        ev1.record()
        torch.cuda.synchronize()
        t_h += ev0.elapsed_time(ev1)
        H_in.append(hs[0])
        H_mid.append(hs[1])
    return gu, H_in, dn, H_mid, t_h


def run_experts(args):
    """--workload c4: one step = the 128 experts' gate_up_proj and down_proj through quantize_experts with PACK
    (per-expert rotation, factors and refit; the row quantizer of all experts of one shape in shared Viterbi
    launches) plus every expert's .ltq slice packing."""
    import torch
    from ltq_amd import liqk, ltq_file, moe, tcq_proto
    from ltq_amd.formats import TCQ_CONFIG, make_format
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    n_exp = args.experts or C4_EXPERTS
    gu, H_in, dn, H_mid, t_h = prepare_experts(dev, n_exp)
    f = make_format(C4_FORMAT)
    seeds_gu = [moe.expert_seed(0, f"gu{e}") for e in range(n_exp)]
    seeds_dn = [moe.expert_seed(0, f"dn{e}") for e in range(n_exp)]

    def step():
        liqk.PACK = {}
        try:
            out_gu, fl_gu = moe.quantize_experts(gu, H_in, C4_FORMAT, seeds_gu, damp=DAMP / 10)
            out_dn, fl_dn = moe.quantize_experts(dn, H_mid, C4_FORMAT, seeds_dn, damp=DAMP / 10)
        finally:
            liqk.PACK = None
        packed = [ltq_file.pack_slice_device(m["idx"], m["gi"], f) for m in fl_gu + fl_dn]
        return out_gu, out_dn, packed

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    tcq_proto.LAUNCH_EVENTS, tcq_proto.LAUNCH_SAMPLE, tcq_proto._launch_count = [], 1, 0
    tcq_proto.EVENT_FACTORY = DeviceEvent
    t0 = time.perf_counter()
    for _ in range(args.steps):
        out_gu, out_dn, packed = step()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    evs, tcq_proto.LAUNCH_EVENTS = tcq_proto.LAUNCH_EVENTS, None
    t_vit, ops, n_launch = viterbi_event_totals(evs)
    achieved = ops / t_vit / 1e12
    weights = n_exp * (2 * C4_INTER * C4_HIDDEN + C4_HIDDEN * C4_INTER)
    value = weights / (dt / args.steps) / 1e6
    rel = [r for _, _, r in out_gu + out_dn]
    res = {
        "metric": f"Mweights/s quantized (C4 MoE expert batch: {n_exp} experts x gate_up 1536x2048 + down 2048x768, "
                  f"K=3 D4 16-subset, 4 gain candidates) on 1 GPU; % VALU ACS roofline",
        "value": round(value, 3), "unit": "Mweights/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(dt / args.steps * 1e3, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32",
        "data": "synthetic, generated on the device (Student-t(5)*0.02 bf16 experts, per-expert Hessians from 256 "
                "N(0,1) bf16 activation rows; seeds 10+e / 20000+e)",
        "config": {"workload": f"C4 {n_exp} experts: gate_up_proj [1536, 2048] and down_proj [2048, 768] per expert, "
                               f"{C4_FORMAT} (K=3 D4, masks 359/40/475, h=3, n_cand=4) tail-biting tb_window=32, "
                               f"damping 0.2, LDLQ on; one step = quantize_experts for both shapes (one Viterbi "
                               f"launch per sub-block over all experts' tiles) with PACK + .ltq slices",
                   "format": C4_FORMAT, "experts": n_exp, "parallelism": "single GPU"},
        "roofline": {"bound": "valu", "timed_on": "a HIP start / stop event pair carried by each Viterbi "
                                                  "launch of the timed steps (hipExtLaunchKernelGGL)",
                     "achieved": round(achieved, 3), "peak": VALU_PEAK_TOPS,
                     "unit": "TFLOP/s (fp32 VALU lane-ops/s x 1e-12)", "frac": round(achieved / VALU_PEAK_TOPS, 4),
                     "traffic": None, "kernel": "tcq_viterbi_kernel<10,2,2,16,1>",
                     "viterbi_ms_per_step": round(t_vit / args.steps * 1e3, 2),
                     "viterbi_launches_per_step": n_launch // args.steps},
        "breakdown": {"mweights_s_viterbi": round(weights / (t_vit / args.steps) / 1e6, 3),
                      "h_build_ms": round(t_h, 2), "proxy_rel_loss_mean": round(sum(rel) / len(rel), 6),
                      "packed_bytes": int(sum(p.numel() for p in packed))},
    }
    print(json.dumps(res), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU baseline sample (0 = skip)")
    ap.add_argument("--cols", type=int, default=K_COLS, help="matrix columns (profiling runs may use fewer)")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="profiling runs: first copy this many MiB device-to-device (a known-size kernel that "
                         "calibrates the FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--workload", choices=("c3", "c4", "c5"), default="c3",
                    help="c3: the headline matrix quantizer (default); c4: the MoE expert batch; c5: the ring table "
                         "(extra lines on request)")
    ap.add_argument("--experts", type=int, default=0, help="c4: number of experts (default 128)")
    ap.add_argument("--rows", type=int, default=0, help="c5: table rows (default 262144)")
    ap.add_argument("--format", default="", help="c5: ring format (default TCQ375X, K=4 D4; TCQ4X as published)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the quantizer is row-sharded with no exchange on the hot path, "
              "and this build runs and reports a single MI355X (--gpus 1).", file=sys.stderr)
        sys.exit(2)
    if args.cols % 256 or args.cols <= 0:
        sys.exit("--cols must be a positive multiple of 256")
    if args.workload == "c5":
        return run_rings(args)
    if args.workload == "c4":
        return run_experts(args)

    import torch
    from ltq_amd import liqk, ltq_file, tcq_proto
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
    W, H, h_build = prepare(dev, cols=args.cols)
    rows, cols = W.shape
    stream = torch.cuda.current_stream()

    def step():
        """W (bf16, HBM) and H -> rotation, suh, factors, row scale, LDLQ + Viterbi, refit, packed .ltq slice."""
        liqk.PACK = {}
        try:
            q, _, rel = liqk.quantize_matrix_liqk_v2(W, H, FORMAT, damp=DAMP / 10)
            pm = liqk.PACK["matrix"]
        finally:
            liqk.PACK = None
        packed = ltq_file.pack_slice_device(pm["idx"], pm["gi"], f)
        liqk._mark("pack")
        return packed, pm, q, rel

    timer = KernelTimer()
    timer.install()
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # stage marks every step; Viterbi launch events on one sub-block in 17 (both passes; 17 is prime to the 16
    # sub-blocks of a column block, whose first one follows the inter-block update and runs ~0.6 us slower, so
    # every position is sampled alike); events carried by the rotation, row-scale, pack and LDLQ-update launches
    timer.active = True
    liqk.STAGE_EVENTS, tcq_proto.LAUNCH_EVENTS = [], []
    tcq_proto.EVENT_FACTORY = DeviceEvent
    tcq_proto.LAUNCH_SAMPLE, tcq_proto._launch_count = 17, 0
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        packed, pm, q, rel = step()
    e1.record(stream)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    stage_ev, launch_ev = liqk.STAGE_EVENTS, tcq_proto.LAUNCH_EVENTS
    liqk.STAGE_EVENTS = tcq_proto.LAUNCH_EVENTS = None
    timer.active = False
    kernels = timer.summary(args.steps)
    timer.uninstall()

    ms_step = dt / args.steps * 1e3
    weights = rows * cols
    value = weights / (dt / args.steps) / 1e6
    # stage durations (per step, ms): consecutive marks start, rotation, factor, rows, refit, pack
    stages = {}
    for i in range(1, len(stage_ev)):
        name, ev = stage_ev[i]
        if name == "start":
            continue
        stages[name] = stages.get(name, 0.0) + stage_ev[i - 1][1].elapsed_time(ev) / args.steps
    # one record per sampled sub-block: both passes (2 * tb_window and 256 steps over rows / 16 tiles), an event
    # pair on each launch
    secs, ops_timed, n_timed = viterbi_event_totals(launch_ev)
    avg = secs / n_timed
    n_launch = 2 * (cols // 256) * 16
    t_vit = avg * n_launch
    ntile = rows // 16
    ops = ops_timed / n_timed
    achieved = ops / avg / 1e12
    traffic = read_traffic()
    t_mat = sum(stages.get(k, 0.0) for k in ("rotation", "rows", "pack")) * 1e-3
    out = {
        "metric": "Mweights/s quantized (K=3 D4, 4096x14336) on 1 GPU; % VALU ACS roofline",
        "value": round(value, 3), "unit": "Mweights/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_step, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic, generated on the device (Student-t(5)*0.02 bf16 weights, 143 outlier "
                                "columns x20; H from 2048 N(0,1) bf16 activation rows; seeds 0/1/2)",
        "config": {"workload": f"C3 down_proj {rows}x{cols} {FORMAT} (K=3 D4, nl=8, h=2) tail-biting "
                               f"tb_window={TB_WINDOW}, damping {DAMP} mean(diag H_rot), LDLQ on: one step = "
                               f"quantize_matrix_liqk_v2 with PACK (rotation, factors, row scale, "
                               f"{cols // 256 * 16} two-pass Viterbi sub-blocks of {ntile} tiles, LDLQ, refit) + "
                               f".ltq slice packing",
                   "format": FORMAT, "rows": rows, "cols": cols, "parallelism": "single GPU"},
        "roofline": {"bound": "valu", "timed_on": "a HIP start / stop event pair carried by each of the two Viterbi launches of "
                                  "one sub-block in 17 (hipExtLaunchKernelGGL)", "achieved": round(achieved, 3), "peak": VALU_PEAK_TOPS,
                     "unit": "TFLOP/s (fp32 VALU lane-ops/s x 1e-12)", "frac": round(achieved / VALU_PEAK_TOPS, 4),
                     "traffic": traffic, "kernel": "tcq_viterbi_kernel<10,2,2,8,1>",
                     "avg_launch_us": round(avg * 1e6, 2), "lane_ops_per_launch": ops},
        "breakdown": {"stages_ms": {k: round(v, 3) for k, v in stages.items()},
                      "t_mat_ms": round(t_mat * 1e3, 3), "mweights_s_t_mat": round(weights / t_mat / 1e6, 3),
                      "t_vit_ms": round(t_vit * 1e3, 3), "mweights_s_viterbi": round(weights / t_vit / 1e6, 3),
                      "viterbi_launches_per_step": n_launch, "viterbi_launches_timed": n_timed,
                      "proxy_rel_loss": round(rel, 6),
                      "packed_bytes": int(packed.numel())},
        "h_build": h_build,
        "hbm": {k: v for k, v in kernels.items() if k != "ldlq_update"},
        "ldlq_update": kernels.get("ldlq_update"),
    }
    if args.cpu_seconds > 0:
        inputs = block_inputs(W, H)
        out["cpu_baseline"] = cpu_baseline_torch(inputs, args.cpu_seconds, (cols // 256) * 16)
        out["cpu_baseline_c_port"] = cpu_baseline_port(inputs, min(args.cpu_seconds, 10.0))
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
