"""Benchmark: BCJR fwd+bwd trellis state-updates/s on one MI355X.

Workload (default): the single-tile kernel config -- L=16 (65,536 states), k=2,
V=1, 256 steps, 4,096 sequences (one 1024x1024 float32 N(0,1) matrix in 16x16
tiles), 3INST codebook, T=0.1.  One step = forward (soft codewords) + backward
(gradient wrt the sequences) of the BCJR node over the whole batch, with inputs
resident in HBM.  State-updates per step = 4 sweeps (alpha, beta and the two
adjoint sweeps) x B x N x 2^L cells; recompute sweeps are not counted.

Also reported:
  * per-kernel durations from HIP events on the launch stream;
  * the roofline of the step (both launches) against the measured v_exp_f32
    issue rate, counting 5 + 2 * 2^-kV algorithmic transcendentals per cell
    (3 + 2 * 2^-kV of them belong to the soft forward, the other 2 to the
    gradient);
  * HBM bytes per step from the committed counter summary
    (profiles/bcjr_tile_hbm_traffic.txt), when present;
  * seconds per Llama-3.2-1B decoder-layer QAT step (237,568 sequences): a
    4,096-sequence fwd+bwd timed at each per-tensor temperature of that layer,
    plus the Viterbi pack of every tile and the random Hadamard transforms
    around each weight tensor;
  * dequantization of one Llama-3.2-1B layer from the packed 2-bit format
    (bcjr_dequant + inverse RHT per tensor), with the dequant kernel's HBM
    roofline;
  * seconds per Llama-3.2-1B MLP-block QAT step (196,608 sequences at T), from
    the timed step;
  * the reference QAT shape (L=16, V=2, N=128, HYB) as a secondary config;
  * the expert-batched dispatch on OLMoE-1B-7B expert shapes against the
    per-weight loop, and the 64-expert layer time it implies;
  * the CPU oracle (C/OpenMP) timed on a bounded sample of the same workload.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--config tile|cpu]
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "quant-2bit_amd"))
sys.path.insert(0, ROOT)


# Algorithmic transcendentals per cell (exp2/log2), structure-aware count:
#   soft pass: alpha-LSE exp + beta-LSE exp + marginal exp + one log per 2^kV group per sweep
#   fwd+grad : the soft pass plus one exp per cell for each adjoint sweep
def trans_per_cell_soft(kV):
    return 3.0 + 2.0 * 2.0 ** (-kV)


def trans_per_cell_grad(kV):
    return 5.0 + 2.0 * 2.0 ** (-kV)


# Llama-3.2-1B decoder layer: (rows, cols, T) per weight tensor, 256-weight tiles.
LAYER_TENSORS = (("q", 2048, 2048, 0.05), ("k", 512, 2048, 0.08), ("v", 512, 2048, 0.12),
                 ("o", 2048, 2048, 0.2), ("gate", 8192, 2048, 0.3), ("up", 8192, 2048, 0.4),
                 ("down", 2048, 8192, 0.5))
LAYER_SEQS = sum(r * c // 256 for _, r, c, _ in LAYER_TENSORS)  # 237,568
MLP_SEQS = 3 * 8192 * 2048 // 256  # gate, up, down: 196,608
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "bcjr_tile_hbm_traffic.txt")
CALIB_BYTES = 256 << 20


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", default="tile", choices=["tile", "cpu"])
    ap.add_argument("--T", type=float, default=0.1)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample", type=int, default=256, help="sequences in the CPU baseline sample")
    ap.add_argument("--no-layer", action="store_true", help="skip the whole-layer steps (single-tile and reference QAT shapes)")
    ap.add_argument("--no-dequant", action="store_true", help="skip the dequant (on-disk format) leg")
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip the reference QAT shape (L=16, V=2, N=128, HYB) leg")
    ap.add_argument("--experts", type=int, default=2,
                    help="OLMoE experts in the expert-batched dispatch leg (0 skips it)")
    return ap.parse_args()


def measure_peaks(torch, dev):
    """v_exp_f32 / v_log_f32 / v_fma_f32 issue rates (per second, whole chip)."""
    import bcjr
    lib = ctypes.CDLL(os.path.join(os.path.dirname(bcjr.LIB_PATH), "libbcjr_peak.so"))
    lib.bcjr_peak_launch.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                                     ctypes.c_int, ctypes.c_void_p]
    chains = lib.bcjr_peak_chains()
    n_cu = torch.cuda.get_device_properties(dev).multi_processor_count
    blocks = n_cu * 16  # 16 waves of 64 per CU (4 per SIMD)
    sink = torch.empty(blocks * 256, device=dev)
    stream = torch.cuda.current_stream(dev)
    out = {}

    def run(kind, K, iters):
        rc = lib.bcjr_peak_launch(kind, K, sink.data_ptr(), blocks, iters, ctypes.c_void_p(stream.cuda_stream))
        assert rc == 0, rc

    for name, kind, K, per_iter in (("exp", 0, 0, 1), ("log", 1, 0, 1), ("fma", 2, 0, 1),
                                    ("exp+2fma", 3, 2, 1), ("exp+4fma", 3, 4, 1)):
        iters = 4096
        run(kind, K, 64)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        run(kind, K, iters)
        e1.record(stream)
        torch.cuda.synchronize(dev)
        sec = e0.elapsed_time(e1) / 1e3
        ops = blocks * 256.0 * chains * iters * per_iter
        out[name] = {"per_s": ops / sec, "ms": sec * 1e3}
    return out


def cpu_baseline(seq, g, cb_np, T, L, kV, sample):
    import numpy as np
    import oracle
    threads = len(os.sched_getaffinity(0))
    threads = min(threads, 16)
    oracle.num_threads(threads)
    s = seq[:sample]
    gg = g[:sample]
    t0 = time.perf_counter()
    oracle.bcjr_forward(s, cb_np, T, L, kV, nthreads=threads)
    oracle.bcjr_backward(s, cb_np, T, L, kV, gg, nthreads=threads)
    dt = time.perf_counter() - t0
    cells = sample * s.shape[1] * (1 << L)
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": 4.0 * cells / dt, "unit": "state-updates/s", "cores": threads, "kind": "port",
            "seconds": dt,
            "sample": f"{sample} of the workload's sequences, fwd+bwd, C/OpenMP float64 oracle "
                      f"(oracle/bcjr_oracle.c), {cpu_model}"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the path shards "
              "across GPUs by sequences with no collective inside BCJR.", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch
    import bcjr
    from bcjr import ops

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.config == "tile":
        L, k, V, N, B, kind = 16, 2, 1, 256, 4096, "3inst"
        workload = "single-tile: L=16 k=2 V=1 N=256 B=4096 (1024x1024 matrix), 3INST, T=%g" % args.T
    else:
        L, k, V, N, B, kind = 12, 2, 1, 256, 128, "1mad"
        workload = "cpu-config: L=12 k=2 V=1 N=256 B=128, 1MAD, T=%g" % args.T
    kV = k * V
    rng = np.random.default_rng(0)
    seq_np = rng.standard_normal((B, N, V)).astype(np.float32)
    g_np = np.random.default_rng(1).standard_normal((B, N, V)).astype(np.float32)
    cb = bcjr.make_3inst_codebook(L, dev) if kind == "3inst" else bcjr.make_1mad_codebook(L, dev)
    x = torch.tensor(seq_np, device=dev)
    g = torch.tensor(g_np, device=dev)
    spec, _ = bcjr.codes.resolve_codebook(cb, L, k, V, dev)

    def step():
        xs = x.detach().requires_grad_(True)
        soft, _ = bcjr.bcjr_forward_backward(xs, cb, args.T, L=L, k=k, V=V)
        soft.backward(g)
        return xs.grad

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - t0
    ms_step = wall / args.steps * 1e3
    cells = float(B) * N * (1 << L)
    value = 4.0 * cells / (wall / args.steps)

    # Per-kernel durations (HIP events on the stream the kernels run on).
    stream = torch.cuda.current_stream(dev)
    reps = max(2, min(args.steps, 5))
    t_f, t_b = [], []
    for _ in range(reps):
        e = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
        e[0].record(stream)
        ops.forward(spec, x, args.T, None)
        e[1].record(stream)
        e[2].record(stream)
        ops.backward(spec, x, args.T, None, g)
        e[3].record(stream)
        torch.cuda.synchronize(dev)
        t_f.append(e[0].elapsed_time(e[1]) / 1e3)
        t_b.append(e[2].elapsed_time(e[3]) / 1e3)
    fwd_s, bwd_s = sum(t_f) / reps, sum(t_b) / reps
    # The forward with the fused marginal entropy (entropy_diagnostic over every tile).
    t_h = []
    for _ in range(reps):
        e = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        e[0].record(stream)
        ops.forward_entropy(spec, x, args.T, None)
        e[1].record(stream)
        torch.cuda.synchronize(dev)
        t_h.append(e[0].elapsed_time(e[1]) / 1e3)
    ent_s = sum(t_h) / reps

    peaks = measure_peaks(torch, dev)
    exp_peak = peaks["exp"]["per_s"]
    # Roofline of one QAT step (forward + backward launches).
    step_s = fwd_s + bwd_s
    per_cell = trans_per_cell_grad(kV)
    achieved = per_cell * cells / step_s
    traffic = read_traffic()
    roofline = {
        "bound": "valu_exp", "kernel": "bcjr_fwd_kernel+bcjr_bwd_kernel",
        "achieved": achieved / 1e12, "peak": exp_peak / 1e12, "unit": "Texp/s",
        "frac": achieved / exp_peak, "traffic": traffic,
        "per_cell": per_cell, "cells": cells, "launch_s": step_s,
    }
    if traffic is not None:
        roofline["hbm_GB_s"] = traffic / step_s / 1e9
        roofline["hbm_frac"] = traffic / step_s / 8e12
    soft_pc, grad_pc = trans_per_cell_soft(kV), trans_per_cell_grad(kV) - trans_per_cell_soft(kV)
    kernels = {
        "bcjr_fwd_kernel": {"ms": fwd_s * 1e3, "trans_per_cell": soft_pc,
                            "frac": soft_pc * cells / fwd_s / exp_peak},
        "bcjr_bwd_kernel": {"ms": bwd_s * 1e3, "trans_per_cell": grad_pc,
                            "frac": grad_pc * cells / bwd_s / exp_peak},
        "bcjr_fwd_kernel (marginal entropy)": {"ms": ent_s * 1e3, "vs_forward": ent_s / fwd_s},
    }
    layer = None
    if args.config == "tile" and not args.no_layer:
        layer = layer_estimate(torch, bcjr, ops, cb, L, k, V, N, B, dev)
    secondary = None
    if args.config == "tile" and not args.no_secondary:
        secondary = secondary_config(torch, bcjr, ops, dev, exp_peak, args.T, whole_layer=not args.no_layer)
    dequant = None
    if args.config == "tile" and not args.no_dequant:
        dequant = dequant_estimate(torch, bcjr, ops, dev)
    experts = None
    if args.config == "tile" and args.experts > 0:
        experts = experts_estimate(torch, bcjr, dev, args.experts, args.T)
    calibration_copy(torch, dev)
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(seq_np, g_np, cb.cpu().numpy(), args.T, L, kV, min(args.cpu_sample, B))

    line = {
        "metric": "BCJR fwd+bwd state-updates/sec (L=16,k=2); s per Llama-1B layer QAT step",
        "value": value, "unit": "state-updates/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms_step, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic N(0,1) sequences (seed 0), upstream gradient N(0,1) (seed 1)",
        "config": {"workload": workload, "L": L, "k": k, "V": V, "N": N, "B": B, "code": kind, "T": args.T},
        "layer_step_s": layer["seconds"] if layer else None,
        # Llama-3.2-1B MLP block (gate/up 8192x2048, down 2048x8192: 196,608 sequences) at T
        "mlp_block_step_s": (ms_step / 1e3) * MLP_SEQS / B if args.config == "tile" else None,
        "layer": layer,
        "roofline": roofline, "kernels": kernels,
        "secondary": secondary, "dequant": dequant, "experts": experts,
        "peaks_per_s": {k_: v["per_s"] for k_, v in peaks.items()},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def read_traffic():
    """HBM bytes per step (forward + backward launch) from the committed counter
    summary: the line 'traffic_bytes_per_step: <float>'."""
    try:
        for line in open(TRAFFIC_FILE):
            if line.startswith("traffic_bytes_per_step:"):
                return float(line.split(":", 1)[1])
    except (OSError, ValueError):
        pass
    return None


def layer_estimate(torch, bcjr, ops, cb, L, k, V, N, B, dev):
    """Seconds per Llama-3.2-1B decoder-layer QAT step, measured whole (every
    tensor's sequences in one forward and one backward launch with per-sequence
    T, one Viterbi launch, four RHTs per tensor), beside the per-tensor
    breakdown: one forward + backward over a B-sequence batch timed at each
    tensor's temperature, scaled by that tensor's sequence count."""
    spec, _ = bcjr.codes.resolve_codebook(cb, L, k, V, dev)
    x = torch.randn(B, N, V, device=dev, generator=torch.Generator(dev).manual_seed(2))
    g = torch.randn(B, N, V, device=dev, generator=torch.Generator(dev).manual_seed(3))
    stream = torch.cuda.current_stream(dev)
    total, per = 0.0, {}
    for name, rows, cols, T in LAYER_TENSORS:
        ops.forward(spec, x, T, None)
        ops.backward(spec, x, T, None, g)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        ops.forward(spec, x, T, None)
        ops.backward(spec, x, T, None, g)
        e1.record(stream)
        torch.cuda.synchronize(dev)
        sec = e0.elapsed_time(e1) / 1e3 * (rows * cols // 256) / B
        per[name] = {"T": T, "sequences": rows * cols // 256, "seconds": sec}
        total += sec
    # The T -> 0 Viterbi pack of every tile (walks, 2-bit bitstream) after the soft pass.
    _, table = bcjr.codes.resolve_codebook(cb, L, k, V, dev)
    ops.viterbi(spec, x, table)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    ops.viterbi(spec, x, table)
    e1.record(stream)
    torch.cuda.synchronize(dev)
    vit_batch_s = e0.elapsed_time(e1) / 1e3
    vit = vit_batch_s * LAYER_SEQS / B
    # Random Hadamard transforms around each tensor's quantizer: RHT and its
    # inverse in the forward, their adjoints (the same two transforms) in the
    # backward.  Algorithmic bytes: one read and one write of the matrix.
    rht_s, rht_rates = 0.0, {}
    for name, rows, cols, _ in LAYER_TENSORS:
        Wm = torch.randn(rows, cols, device=dev)
        sl = torch.ones(rows, device=dev)
        sr = torch.ones(cols, device=dev)
        bcjr.apply_inverse_rht_gpu(bcjr.apply_rht_gpu(Wm, sl, sr), sl, sr)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        Wt = bcjr.apply_rht_gpu(Wm, sl, sr)
        e1.record(stream)
        torch.cuda.synchronize(dev)
        one = e0.elapsed_time(e1) / 1e3
        rht_s += 4 * one
        rht_rates[name] = {"ms": one * 1e3, "GB_s": 8.0 * rows * cols / one / 1e9}
        del Wt
    # The same step measured whole: every tensor's sequences in one forward and
    # one backward launch, each sequence carrying its tensor's T, then one
    # Viterbi launch over all of them (237,568 sequences, ~1 GB of inputs and
    # outputs).
    del x, g
    Ts = torch.cat([torch.full((rows * cols // 256,), T, device=dev) for _, rows, cols, T in LAYER_TENSORS])
    X = torch.randn(LAYER_SEQS, N, V, device=dev, generator=torch.Generator(dev).manual_seed(4))
    G = torch.randn(LAYER_SEQS, N, V, device=dev, generator=torch.Generator(dev).manual_seed(5))
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    ev[0].record(stream)
    ops.forward(spec, X, Ts, None)
    ops.backward(spec, X, Ts, None, G)
    ev[1].record(stream)
    ops.viterbi(spec, X, table)
    ev[2].record(stream)
    torch.cuda.synchronize(dev)
    meas_soft = ev[0].elapsed_time(ev[1]) / 1e3
    meas_vit = ev[1].elapsed_time(ev[2]) / 1e3
    del X, G
    cells = float(LAYER_SEQS) * N * (1 << L)
    return {"seconds": meas_soft + meas_vit + rht_s,
            "measured": {"soft_seconds": meas_soft, "viterbi_seconds": meas_vit,
                         "state_updates_per_s": 4.0 * cells / meas_soft,
                         "note": "one forward and one backward launch over all %d sequences with per-sequence T, "
                                 "one Viterbi launch over all of them, plus the four RHTs per tensor" % LAYER_SEQS},
            "estimate_seconds": total + vit + rht_s, "soft_seconds": total, "viterbi_seconds": vit,
            "rht_seconds": rht_s, "rht_per_tensor": rht_rates,
            "viterbi_ms_per_%d_sequences" % B: vit_batch_s * 1e3,
            "sequences": LAYER_SEQS, "tensors": per,
            "state_updates_per_s": 4.0 * cells / total,
            "note": "seconds: the measured whole-layer step; estimate_seconds: fwd+bwd per tensor timed on a "
                    "%d-sequence batch at that tensor's T, scaled by its sequence count, plus one Viterbi pack of "
                    "every tile and four random Hadamard transforms per tensor" % B}


def secondary_config(torch, bcjr, ops, dev, exp_peak, T, B=4096, whole_layer=True):
    """The reference QAT shape as a secondary config: L=16, k=2, V=2 (kV=4), N=128
    steps, HYB codebook (random 2^9 x 2 LUT), B sequences of N(0,1) weights:
    forward + backward of the node, per-launch durations from HIP events, and
    the roofline at 5 + 2 * 2^-4 algorithmic transcendentals per cell."""
    import numpy as np
    L, k, V, N = 16, 2, 2, 128
    lut = np.random.default_rng(3).standard_normal((512, 2)).astype(np.float32)
    cb = bcjr.make_hyb_codebook_gpu(lut, 9, L, dev)
    spec, table = bcjr.codes.resolve_codebook(cb, L, k, V, dev)
    x = torch.randn(B, N, V, device=dev, generator=torch.Generator(dev).manual_seed(4))
    g = torch.randn(B, N, V, device=dev, generator=torch.Generator(dev).manual_seed(5))
    stream = torch.cuda.current_stream(dev)
    ops.forward(spec, x, T, table)
    ops.backward(spec, x, T, table, g)
    reps = 3
    e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    e[0].record(stream)
    for _ in range(reps):
        ops.forward(spec, x, T, table)
    e[1].record(stream)
    for _ in range(reps):
        ops.backward(spec, x, T, table, g)
    e[2].record(stream)
    torch.cuda.synchronize(dev)
    fwd_s = e[0].elapsed_time(e[1]) / 1e3 / reps
    bwd_s = e[1].elapsed_time(e[2]) / 1e3 / reps
    # The hard (T -> 0) pack of the same tiles: the STE path's Viterbi launch.
    ops.viterbi(spec, x, table)
    e[0].record(stream)
    for _ in range(reps):
        ops.viterbi(spec, x, table)
    e[1].record(stream)
    torch.cuda.synchronize(dev)
    vit_s = e[0].elapsed_time(e[1]) / 1e3 / reps
    # A Llama-3.2-1B layer at this shape, measured whole: 237,568 tiles of 128
    # steps in one forward and one backward launch, each tile at its tensor's T
    # (q .05 ... down .5), then one Viterbi launch over all of them.
    del x, g
    layer_soft_s = layer_vit_s = None
    if whole_layer:
        layer_soft_s, layer_vit_s = _secondary_layer(torch, ops, spec, table, dev, N, V, stream, e)
    cells = float(B) * N * (1 << L)
    per_cell = trans_per_cell_grad(k * V)
    return {"workload": "reference QAT shape: L=16 k=2 V=2 (kV=4) N=128 B=%d, HYB, T=%g" % (B, T),
            "fwd_ms": fwd_s * 1e3, "bwd_ms": bwd_s * 1e3, "viterbi_ms": vit_s * 1e3,
            "viterbi_cells_per_s": cells / vit_s,
            "state_updates_per_s": 4.0 * cells / (fwd_s + bwd_s),
            "roofline": {"bound": "valu_exp", "achieved": per_cell * cells / (fwd_s + bwd_s) / 1e12,
                         "peak": exp_peak / 1e12, "unit": "Texp/s",
                         "frac": per_cell * cells / (fwd_s + bwd_s) / exp_peak, "per_cell": per_cell},
            # A Llama-3.2-1B layer at this shape (the reference's own training config: 237,568 tiles of
            # 128 steps, per-tensor T), measured whole: the soft fwd+bwd and one Viterbi pack.  The
            # reference's layer-step wall clocks (whole QAT steps, dominated by its BCJR) are context
            # from its scripts, not a like-for-like measurement.
            "layer_step_s": layer_soft_s + layer_vit_s if whole_layer else None,
            "layer": {"soft_seconds": layer_soft_s, "viterbi_seconds": layer_vit_s,
                      "estimate_at_T_%g_s" % T: (fwd_s + bwd_s + vit_s) * LAYER_SEQS / B},
            "reference_layer_step_s_context": {"H100 SXM": 1644, "RTX 4080 Laptop": 4920,
                                               "source": "scripts/vast_resume_llama.sh:13-14, "
                                                         "scripts/rung_matched_l4.sh:8"}}


def _secondary_layer(torch, ops, spec, table, dev, N, V, stream, e):
    """Soft fwd+bwd seconds and Viterbi seconds of one whole Llama-3.2-1B layer at
    the reference QAT shape (one launch each, per-sequence T)."""
    Ts = torch.cat([torch.full((rows * cols // 256,), Tl, device=dev) for _, rows, cols, Tl in LAYER_TENSORS])
    X = torch.randn(LAYER_SEQS, N, V, device=dev, generator=torch.Generator(dev).manual_seed(6))
    G = torch.randn(LAYER_SEQS, N, V, device=dev, generator=torch.Generator(dev).manual_seed(7))
    e[0].record(stream)
    ops.forward(spec, X, Ts, table)
    ops.backward(spec, X, Ts, table, G)
    e[1].record(stream)
    ops.viterbi(spec, X, table)
    e[2].record(stream)
    torch.cuda.synchronize(dev)
    return e[0].elapsed_time(e[1]) / 1e3, e[1].elapsed_time(e[2]) / 1e3


def dequant_estimate(torch, bcjr, ops, dev):
    """Dequantization of a Llama-3.2-1B decoder layer from the packed 2-bit format
    (HYB L=16, k=2, V=2): bcjr_dequant per tensor (walk replay + codebook +
    untiling + scale into the rotated-basis matrix) and the inverse RHT after it.
    Algorithmic bytes of bcjr_dequant per weight: a 4-byte write plus k/8 bytes
    of packed bitstream (2 bits); the kernel is HBM-bound."""
    import numpy as np
    lut = np.random.default_rng(5).standard_normal((512, 2)).astype(np.float32)
    cb = bcjr.make_hyb_codebook_gpu(lut, 9, 16, dev)
    spec = ops.Spec(16, 2, 2, ops.CODE_HYB, 9)
    stream = torch.cuda.current_stream(dev)
    per, tot_k, tot_r, tot_bytes = {}, 0.0, 0.0, 0.0
    for name, rows, cols, _ in LAYER_TENSORS:
        B = rows * cols // 256
        g = torch.Generator(dev).manual_seed(rows + cols)
        packed = torch.randint(0, 256, (B, 64), dtype=torch.uint8, device=dev, generator=g)
        start = torch.randint(0, 1 << 16, (B,), dtype=torch.int32, device=dev, generator=g)
        sl = torch.ones(rows, device=dev)
        sr = torch.ones(cols, device=dev)
        W = ops.dequant(spec, start, cb._bcjr_lut, rows, cols, 16, 16, 0.02, packed=packed)
        bcjr.apply_inverse_rht_gpu(W, sl, sr)
        reps = 5
        e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        e[0].record(stream)
        for _ in range(reps):
            W = ops.dequant(spec, start, cb._bcjr_lut, rows, cols, 16, 16, 0.02, packed=packed)
        e[1].record(stream)
        for _ in range(reps):
            Wh = bcjr.apply_inverse_rht_gpu(W, sl, sr)
        e[2].record(stream)
        torch.cuda.synchronize(dev)
        kd = e[0].elapsed_time(e[1]) / 1e3 / reps
        kr = e[1].elapsed_time(e[2]) / 1e3 / reps
        nbytes = rows * cols * (4.0 + 2.0 / 8.0) + 4.0 * B
        per[name] = {"dequant_us": kd * 1e6, "inverse_rht_us": kr * 1e6, "GB_s": nbytes / kd / 1e9}
        tot_k += kd
        tot_r += kr
        tot_bytes += nbytes
        del W, Wh
    # per launch, on the largest tensor (gate: 8192 x 2048, 16.8M weights)
    big = max(LAYER_TENSORS, key=lambda t: t[1] * t[2])
    achieved = big[1] * big[2] * 4.25 / (per[big[0]]["dequant_us"] * 1e-6)
    return {"layer_seconds": tot_k + tot_r, "dequant_seconds": tot_k, "inverse_rht_seconds": tot_r,
            "layer_GB_s": tot_bytes / tot_k / 1e9,
            "roofline": {"bound": "hbm", "kernel": "bcjr_dequant_t16_kernel<4,2,HYB,packed>",
                         "tensor": big[0], "achieved": achieved / 1e9, "peak": 8000.0, "unit": "GB/s",
                         "frac": achieved / 8e12, "bytes_per_weight": 4.25},
            "tensors": per,
            "note": "packed 2-bit bitstreams of every tensor of one Llama-3.2-1B layer, HYB L=16 k=2 V=2"}


def experts_estimate(torch, bcjr, dev, E, T):
    """Expert-batched dispatch on OLMoE-1B-7B expert shapes (gate 1024x2048,
    up 1024x2048, down 2048x1024 per expert; N(0,1) weights times a lognormal
    (sigma 0.5) scale per expert; L=16, k=2, V=1, 3INST): E experts' 3E weights
    soft-quantized forward + backward in one bcjr_quantize_experts call, against
    one bcjr_quantize_weight per weight (the reference's per-expert loop).  The
    64-expert layer time is the batched time scaled by 64 / E."""
    import numpy as np
    cb = bcjr.make_3inst_codebook(16, dev)
    kw = dict(L=16, k=2, V=1)
    shapes = [(1024, 2048), (1024, 2048), (2048, 1024)] * E
    scales = np.exp(np.random.default_rng(7).normal(0.0, 0.5, E)).repeat(3)
    g = torch.Generator(dev).manual_seed(11)
    Ws = [torch.randn(s, device=dev, generator=g) * float(sc) for s, sc in zip(shapes, scales)]
    gs = [torch.randn(s, device=dev, generator=g) for s in shapes]
    sl = [torch.ones(s[0], device=dev) for s in shapes]
    sr = [torch.ones(s[1], device=dev) for s in shapes]
    # small warm-up of both paths (plans, LUT upload)
    w0 = [torch.randn(64, 64, device=dev, requires_grad=True)]
    o = bcjr.bcjr_quantize_experts(w0, [torch.ones(64, device=dev)], [torch.ones(64, device=dev)], cb, T, **kw)
    o[0].sum().backward()

    def batched():
        lat = [w.detach().requires_grad_(True) for w in Ws]
        outs = bcjr.bcjr_quantize_experts(lat, sl, sr, cb, T, **kw)
        torch.autograd.backward(outs, gs)
        return lat

    def loop():
        lat = [w.detach().requires_grad_(True) for w in Ws]
        for w, a, b, gg in zip(lat, sl, sr, gs):
            bcjr.bcjr_quantize_weight(w, a, b, cb, T, **kw).backward(gg)
        return lat

    res = {}
    for name, fn in (("batched", batched), ("loop", loop)):
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize(dev)
        res[name] = time.perf_counter() - t0
    seqs = sum(r * c // 256 for r, c in shapes)
    return {"experts": E, "weights": 3 * E, "sequences": seqs, "batched_seconds": res["batched"],
            "loop_seconds": res["loop"], "speedup": res["loop"] / res["batched"],
            "layer_64_experts_seconds": res["batched"] * 64 / E,
            "layer_64_experts_sequences": seqs * 64 // E,
            "state_updates_per_s": 4.0 * seqs * 256 * 65536 / res["batched"],
            "note": "OLMoE-1B-7B expert shapes (gate, up 1024x2048, down 2048x1024), lognormal per-expert "
                    "scales, 3INST L=16 k=2 V=1, T=%g, forward + backward of the soft quantizer including "
                    "both RHTs" % T}


def calibration_copy(torch, dev):
    """One device-to-device copy of CALIB_BYTES: its FETCH_SIZE / WRITE_SIZE
    counters scale the BCJR kernels' counters to bytes."""
    src = torch.ones(CALIB_BYTES // 4, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize(dev)


if __name__ == "__main__":
    main()
