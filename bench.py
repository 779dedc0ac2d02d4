"""Benchmark: BCJR fwd+bwd trellis state-updates/s and seconds per Llama-3.2-1B
decoder-layer QAT step, on one MI355X.

Workload (default, --config layer): one QAT step of the seven quantized weights
of a Llama-3.2-1B decoder layer -- q/o 2048x2048, k/v 512x2048, gate/up
8192x2048, down 2048x8192 -- with random-init N(0,1) latent weights (seed 0),
per-tensor temperatures q .05, k .08, v .12, o .2, gate .3, up .4, down .5, at
L=16 (65,536 states), k=2, V=1, 16x16 tiles (256 weights, 237,568 tiles), 3INST
codebook.  One step, inputs resident in HBM:
  * the soft quantizer of every weight in one engine call
    (bcjr_quantize_experts: batched RHT, RMS scale, tiles, ONE bcjr_forward
    launch over all 237,568 tiles with per-tile T, untile, inverse RHT),
  * its backward for a fixed upstream gradient (ONE bcjr_backward launch),
  * the T -> 0 Viterbi pack of every tile to the 2-bit bitstream (ONE
    bcjr_viterbi launch).
State-updates per step = 4 sweeps (alpha, beta and the two adjoint sweeps) x
tiles x 256 steps x 2^16 states; recompute sweeps are not counted.  `value` is
that over the whole step (Viterbi and RHTs included).

Also reported:
  * per-kernel durations of the step's three launches from HIP events on the
    launch stream, the roofline of the soft launches against the measured
    v_exp_f32 rate (5 + 2 * 2^-kV algorithmic transcendentals per cell) and
    their HBM traffic from the committed counter summary;
  * secondary: the single-tile config (4,096 tiles, T = 0.1), the reference's
    QAT shape (L=16, V=2, N=128, HYB) on 4,096 tiles with its table-mode timing
    beside it, and on the whole layer (237,568 tiles, whole steps timed), the
    drop-in through bcjr_quantize_weight at chunk_size=8, the dequant of a
    layer from the packed format, and the OLMoE-1B-7B layer's 64 experts
    (1,572,864 tiles) in one expert-batched call against a per-weight loop;
  * cpu_baseline: the reference's eager algorithm (gather + logsumexp +
    autograd, float32) restated in torch (oracle/torch_ref.py), on every host
    core, over a bounded sample of the layer's tiles, extrapolated; beside it
    the CPU-runnable config (L=12, 1MAD, 128 sequences) on a sample and the
    structure-aware C/OpenMP oracle.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--experts E]
                    [--config layer|tile|qat|qat_layer|dequant|cpu]
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

METRIC = "BCJR fwd+bwd state-updates/sec (L=16,k=2); s per Llama-1B layer QAT step"


# Algorithmic transcendentals per cell (exp2/log2), structure-aware count:
#   soft pass: alpha-LSE exp + beta-LSE exp + marginal exp + one log per 2^kV group per sweep
#   fwd+grad : the soft pass plus one exp per cell for each adjoint sweep
def trans_per_cell_soft(kV):
    return 3.0 + 2.0 * 2.0 ** (-kV)


def trans_per_cell_grad(kV):
    return 5.0 + 2.0 * 2.0 ** (-kV)


# Llama-3.2-1B decoder layer: (name, rows, cols, T) per weight tensor, 256-weight tiles.
LAYER_TENSORS = (("q", 2048, 2048, 0.05), ("k", 512, 2048, 0.08), ("v", 512, 2048, 0.12),
                 ("o", 2048, 2048, 0.2), ("gate", 8192, 2048, 0.3), ("up", 8192, 2048, 0.4),
                 ("down", 2048, 8192, 0.5))
LAYER_SEQS = sum(r * c // 256 for _, r, c, _ in LAYER_TENSORS)  # 237,568
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "bcjr_layer_hbm_traffic.txt")
CALIB_BYTES = 256 << 20


def progress(msg):
    """A progress line on stderr (the JSON result goes to stdout)."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--config", default="layer", choices=["layer", "tile", "qat", "qat_layer", "dequant", "cpu"],
                    help="layer: the headline line; tile / qat / dequant: one secondary leg alone (for profiling); "
                         "cpu: the CPU-runnable config on the GPU")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-layer-tiles", type=int, default=7,
                    help="layer tiles in the torch CPU baseline sample (L=16; ~5-15 s each)")
    ap.add_argument("--cpu-config-seqs", type=int, default=128,
                    help="sequences of the L=12 CPU config run by the torch CPU baseline (128 = all)")
    ap.add_argument("--no-secondary", action="store_true", help="skip the secondary workloads")
    ap.add_argument("--experts", type=int, default=64,
                    help="OLMoE experts in the expert-batched dispatch leg (0 skips it)")
    ap.add_argument("--kernels-only", action="store_true",
                    help="time the step's three launches and skip the whole-step timing (profiling runs)")
    return ap.parse_args()


def measure_peaks(torch, dev):
    """v_exp_f32 / v_log_f32 / v_fma_f32 issue rates (per second, whole chip)."""
    import bcjr
    lib = ctypes.CDLL(os.path.join(os.path.dirname(bcjr.LIB_PATH), "libbcjr_peak.so"))
    lib.bcjr_peak_launch.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                                     ctypes.c_int, ctypes.c_void_p]
    chains = lib.bcjr_peak_chains()
    n_cu = torch.cuda.get_device_properties(dev).multi_processor_count
    blocks = n_cu * 16  # 16 blocks of 256 threads per CU: every SIMD as full as residency allows
    sink = torch.empty(blocks * 256, device=dev)
    stream = torch.cuda.current_stream(dev)
    out = {}

    def run(kind, K, iters):
        rc = lib.bcjr_peak_launch(kind, K, sink.data_ptr(), blocks, iters, ctypes.c_void_p(stream.cuda_stream))
        assert rc == 0, rc

    for name, kind, K in (("exp", 0, 0), ("log", 1, 0), ("fma", 2, 0), ("exp+2fma", 3, 2), ("exp+4fma", 3, 4)):
        iters = 4096
        run(kind, K, 64)
        best = None
        for _ in range(3):  # a peak: the fastest of three timed launches
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            run(kind, K, iters)
            e1.record(stream)
            torch.cuda.synchronize(dev)
            sec = e0.elapsed_time(e1) / 1e3
            best = sec if best is None else min(best, sec)
        out[name] = {"per_s": blocks * 256.0 * chains * iters / best, "ms": best * 1e3}
    return out


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def cpu_baseline(args, tiles_np, tiles_T, tiles_g):
    """The reference's eager node (gather + logsumexp + autograd in float32,
    src/bcjr/forward_backward.py:89-232, restated in oracle/torch_ref.py) on all
    host cores: a sample of the layer's tiles (the first tile of each weight in
    turn, at its tensor's T), extrapolated to the layer; the CPU-runnable config
    on a sample (or whole); and the structure-aware C/OpenMP float64 oracle on
    the layer sample."""
    import numpy as np
    import torch
    import oracle
    from oracle.torch_ref import eager_step
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    L, kV = 16, 2
    cb16 = torch.tensor(oracle.codebook(oracle.CODE_3INST, L))
    picks = [i % len(tiles_np) for i in range(args.cpu_layer_tiles)]
    layer_seq_np, layer_g_np, layer_T = tiles_np, tiles_g, tiles_T
    t0 = time.perf_counter()
    for b in picks:
        eager_step(torch.tensor(layer_seq_np[b:b + 1]), cb16, float(layer_T[b]), L, kV,
                   torch.tensor(layer_g_np[b:b + 1]))
    dt = time.perf_counter() - t0
    per_tile = dt / len(picks)
    layer_s = per_tile * LAYER_SEQS
    cells_tile = 256.0 * (1 << L)
    out = {"value": 4.0 * cells_tile / per_tile, "unit": "state-updates/s", "cores": threads, "kind": "port",
           "sample": f"{len(picks)} tiles of the Llama-3.2-1B layer (L=16, k=2, V=1, N=256, 3INST, their tensors' T), "
                     f"forward + gradient of the reference's eager node (gather + logsumexp + per-step checkpoint "
                     f"+ autograd) restated in torch float32 (oracle/torch_ref.py), {threads} threads, {cpu_model()}",
           "seconds": dt, "layer_step_s_extrapolated": layer_s,
           "note": "layer_step_s_extrapolated = seconds per tile x 237,568 tiles (extrapolated, linear in tiles)"}
    # the CPU-runnable config: L=12, 1MAD, T=0.1, N(0,1) seed 0, g seed 1
    Lc, Bc, Nc = 12, 128, 256
    seq_c = np.random.default_rng(0).standard_normal((Bc, Nc, 1)).astype(np.float32)
    g_c = np.random.default_rng(1).standard_normal((Bc, Nc, 1)).astype(np.float32)
    cb12 = torch.tensor(oracle.codebook(oracle.CODE_1MAD, Lc))
    n = min(args.cpu_config_seqs, Bc)
    t0 = time.perf_counter()
    eager_step(torch.tensor(seq_c[:n]), cb12, 0.1, Lc, kV, torch.tensor(g_c[:n]))
    dc = time.perf_counter() - t0
    out["cpu_config"] = {"sequences": n, "seconds": dc, "seconds_all_128": dc * Bc / n,
                         "extrapolated": n < Bc,
                         "state_updates_per_s": 4.0 * n * Nc * (1 << Lc) / dc,
                         "workload": "L=12 k=2 V=1 N=256 B=128, 1MAD, T=0.1, seed 0 (torch float32 eager node)"}
    # the structure-aware C oracle (float64) on the same layer tiles
    oracle.num_threads(threads)
    cbn = cb16.numpy()
    t0 = time.perf_counter()
    for b in picks:
        oracle.bcjr_forward(layer_seq_np[b:b + 1], cbn, float(layer_T[b]), L, kV, nthreads=threads)
        oracle.bcjr_backward(layer_seq_np[b:b + 1], cbn, float(layer_T[b]), L, kV, layer_g_np[b:b + 1],
                             nthreads=threads)
    do = time.perf_counter() - t0
    out["c_oracle"] = {"state_updates_per_s": 4.0 * cells_tile * len(picks) / do,
                       "layer_step_s_extrapolated": do / len(picks) * LAYER_SEQS,
                       "kind": "structure-aware float64 C/OpenMP (oracle/bcjr_oracle.c)"}
    return out


class Layer:
    """The Llama-3.2-1B layer's weights, signs, temperatures and upstream
    gradients, and one QAT step over them.  V = 1 with the 3INST code is the
    headline workload; V = 2 with a HYB table is the reference's own QAT shape
    (N = 128 steps of 2 weights per tile)."""

    def __init__(self, torch, bcjr, dev, V=1, cb=None):
        import numpy as np
        self.torch, self.bcjr, self.dev, self.V = torch, bcjr, dev, V
        self.cb = bcjr.make_3inst_codebook(16, dev) if cb is None else cb
        self.spec, self.table = bcjr.codes.resolve_codebook(self.cb, 16, 2, V, dev)
        rng = np.random.default_rng(0)
        self.W = [torch.tensor(rng.standard_normal((r, c)).astype(np.float32), device=dev)
                  for _, r, c, _ in LAYER_TENSORS]
        gr = np.random.default_rng(1)
        self.G = [torch.tensor(gr.standard_normal((r, c)).astype(np.float32), device=dev)
                  for _, r, c, _ in LAYER_TENSORS]
        self.sl = [torch.tensor(bcjr.make_sign_vector(r, 2 * i), device=dev)
                   for i, (_, r, _, _) in enumerate(LAYER_TENSORS)]
        self.sr = [torch.tensor(bcjr.make_sign_vector(c, 2 * i + 1), device=dev)
                   for i, (_, _, c, _) in enumerate(LAYER_TENSORS)]
        self.T = [T for _, _, _, T in LAYER_TENSORS]
        self.T_tiles = torch.cat([torch.full((r * c // 256,), T, device=dev) for _, r, c, T in LAYER_TENSORS])

    def tiles(self):
        """(237,568, 256 / V, V) rotated, RMS-normalised tiles (what the node sees)."""
        torch, bcjr = self.torch, self.bcjr
        from bcjr.quant import tile_for_viterbi
        out = []
        with torch.no_grad():
            for W, a, b in zip(self.W, self.sl, self.sr):
                Wt = bcjr.apply_rht_gpu(W, a, b)
                s, _ = tile_for_viterbi(Wt / Wt.pow(2).mean().sqrt())
                out.append(s)
        return torch.cat(out).reshape(-1, 256 // self.V, self.V).contiguous()

    def step(self):
        torch, bcjr = self.torch, self.bcjr
        lat = [w.requires_grad_(True) for w in (x.detach() for x in self.W)]
        outs = bcjr.bcjr_quantize_experts(lat, self.sl, self.sr, self.cb, self.T, L=16, k=2, V=self.V)
        torch.autograd.backward(outs, self.G)
        with torch.no_grad():
            packed = bcjr.ops.viterbi(self.spec, self.tiles(), self.table)["packed"]
        return lat, packed


def layer_kernels(torch, ops, layer, dev, reps=1):
    """Durations of the step's three launches over the layer's tiles (HIP events
    on the launch stream), averaged over reps."""
    x = layer.tiles()
    G = torch.randn(x.shape, device=dev, generator=torch.Generator(dev).manual_seed(5))
    stream = torch.cuda.current_stream(dev)
    e = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    tf = tb = tv = 0.0
    for _ in range(reps):
        e[0].record(stream)
        ops.forward(layer.spec, x, layer.T_tiles, layer.table)
        e[1].record(stream)
        ops.backward(layer.spec, x, layer.T_tiles, layer.table, G)
        e[2].record(stream)
        ops.viterbi(layer.spec, x, layer.table)
        e[3].record(stream)
        torch.cuda.synchronize(dev)
        tf += e[0].elapsed_time(e[1]) / 1e3
        tb += e[1].elapsed_time(e[2]) / 1e3
        tv += e[2].elapsed_time(e[3]) / 1e3
    del x, G
    return tf / reps, tb / reps, tv / reps


def read_traffic():
    """HBM bytes of the layer's soft launches (forward + backward) from the
    committed counter summary: the line 'traffic_bytes_per_step: <float>'."""
    try:
        for line in open(TRAFFIC_FILE):
            if line.startswith("traffic_bytes_per_step:"):
                return float(line.split(":", 1)[1])
    except (OSError, ValueError):
        pass
    return None


def tile_config(torch, bcjr, ops, dev, exp_peak, B=4096, T=0.1):
    """The single-tile config: L=16 k=2 V=1 N=256, 4,096 tiles (one 1024x1024
    matrix), 3INST, T=0.1: forward and backward launch durations."""
    cb = bcjr.make_3inst_codebook(16, dev)
    spec, _ = bcjr.codes.resolve_codebook(cb, 16, 2, 1, dev)
    x = torch.randn(B, 256, 1, device=dev, generator=torch.Generator(dev).manual_seed(0))
    g = torch.randn(B, 256, 1, device=dev, generator=torch.Generator(dev).manual_seed(1))
    stream = torch.cuda.current_stream(dev)
    ops.forward(spec, x, T, None)
    ops.backward(spec, x, T, None, g)
    reps = 3
    e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    e[0].record(stream)
    for _ in range(reps):
        ops.forward(spec, x, T, None)
    e[1].record(stream)
    for _ in range(reps):
        ops.backward(spec, x, T, None, g)
    e[2].record(stream)
    torch.cuda.synchronize(dev)
    f = e[0].elapsed_time(e[1]) / 1e3 / reps
    b = e[1].elapsed_time(e[2]) / 1e3 / reps
    # the forward's diagnostics variant with the fused marginal entropy (entropy_diagnostic)
    ops.forward_entropy(spec, x, T, None)
    e[0].record(stream)
    ops.forward_entropy(spec, x, T, None)
    e[1].record(stream)
    torch.cuda.synchronize(dev)
    fe = e[0].elapsed_time(e[1]) / 1e3
    cells = float(B) * 256 * 65536
    return {"workload": "single-tile: L=16 k=2 V=1 N=256 B=4096 (1024x1024 matrix), 3INST, T=0.1",
            "fwd_ms": f * 1e3, "bwd_ms": b * 1e3, "fwd_entropy_ms": fe * 1e3,
            "state_updates_per_s": 4.0 * cells / (f + b),
            "roofline_frac": trans_per_cell_grad(2) * cells / (f + b) / exp_peak}


def qat_shape(torch, bcjr, ops, dev, exp_peak, B=4096, T=0.1):
    """The reference's QAT shape: L=16, k=2, V=2 (kV=4), N=128, HYB codebook
    (random 2^9 x 2 LUT): forward, backward and Viterbi at B tiles, through the
    LUT kernels and through the table kernels (the path an unrecognised
    (2^16, 2) table takes)."""
    import numpy as np
    L, k, V, N = 16, 2, 2, 128
    lut = np.random.default_rng(3).standard_normal((512, 2)).astype(np.float32)
    cb = bcjr.make_hyb_codebook_gpu(lut, 9, L, dev)
    x = torch.randn(B, N, V, device=dev, generator=torch.Generator(dev).manual_seed(4))
    g = torch.randn(B, N, V, device=dev, generator=torch.Generator(dev).manual_seed(5))
    stream = torch.cuda.current_stream(dev)
    cells = float(B) * N * (1 << L)
    res = {"workload": "reference QAT shape: L=16 k=2 V=2 (kV=4) N=128 B=%d, HYB Q=9, T=%g" % (B, T)}
    for mode in ("lut", "table"):
        if mode == "lut":
            spec, table = bcjr.codes.resolve_codebook(cb, L, k, V, dev)
        else:
            spec, table = ops.Spec(L, k, V, ops.CODE_TABLE), cb
        ops.forward(spec, x, T, table)
        ops.backward(spec, x, T, table, g)
        e = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
        e[0].record(stream)
        ops.forward(spec, x, T, table)
        e[1].record(stream)
        ops.backward(spec, x, T, table, g)
        e[2].record(stream)
        ops.viterbi(spec, x, table)
        e[3].record(stream)
        torch.cuda.synchronize(dev)
        f, b, v = (e[i].elapsed_time(e[i + 1]) / 1e3 for i in range(3))
        res[mode] = {"fwd_ms": f * 1e3, "bwd_ms": b * 1e3, "viterbi_ms": v * 1e3,
                     "state_updates_per_s": 4.0 * cells / (f + b),
                     "roofline_frac": trans_per_cell_grad(4) * cells / (f + b) / exp_peak}
    res["table_vs_lut"] = (res["table"]["fwd_ms"] + res["table"]["bwd_ms"]) / (res["lut"]["fwd_ms"] + res["lut"]["bwd_ms"])
    res["note"] = ("lut: the column-walk HYB kernels, which a table made by make_hyb_codebook_gpu (ours or the "
                   "reference's, recognised by content) reaches; table: the table kernels, read c(s) per cell")
    return res


def qat_layer(torch, bcjr, ops, dev, exp_peak, steps=2):
    """The reference's production QAT shape on the whole Llama-3.2-1B decoder
    layer: the same seven weights, per-tensor T and step as the headline, at
    L=16, k=2, V=2 (kV=4, N=128 steps of 2 weights per tile) with a HYB Q=9
    codebook (a random 2^9 x 2 LUT, seed 3) -- the configuration of
    src/qat/ste.py:42-47 and src/bcjr/bcjr_quant.py:146-147 that the reference's
    published step times are quoted on.  One warmup step, then `steps` whole
    steps timed (soft quantizer of every weight + its backward + the Viterbi
    pack), and the three launches timed alone."""
    import numpy as np
    lut = np.random.default_rng(3).standard_normal((512, 2)).astype(np.float32)
    layer = Layer(torch, bcjr, dev, V=2, cb=bcjr.make_hyb_codebook_gpu(lut, 9, 16, dev))
    layer.step()
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    for _ in range(steps):
        layer.step()
    torch.cuda.synchronize(dev)
    step_s = (time.perf_counter() - t0) / steps
    f, b, v = layer_kernels(torch, ops, layer, dev)
    cells = float(LAYER_SEQS) * 128 * 65536
    return {"workload": "Llama-3.2-1B decoder-layer QAT step at the reference's QAT shape: the seven weights "
                        "(237,568 tiles of 256), L=16 k=2 V=2 (kV=4, N=128), HYB Q=9, per-tensor T as the "
                        "headline; RHT + soft fwd + bwd (one launch each) + Viterbi pack",
            "steps": steps, "step_s": step_s, "fwd_s": f, "bwd_s": b, "viterbi_s": v,
            "state_updates_per_s": 4.0 * cells / step_s,
            "roofline_frac": trans_per_cell_grad(4) * cells / (f + b) / exp_peak,
            "reference_context": {
                "h100_sxm_s_per_step": 1644.0, "rtx4080_s_per_step": 4920.0,
                "note": "whole QAT steps of the same layer and shape from the reference's scripts "
                        "(scripts/vast_resume_llama.sh:13-14: 15 steps in ~6.85 h; scripts/rung_matched_l4.sh:8: "
                        "~82 min), which include the model forward/backward and optimizer around BCJR: context, "
                        "not a like-for-like measurement"}}


def drop_in_chunked(torch, bcjr, dev, T=0.3):
    """bcjr_quantize_weight on the gate tensor (8192x2048, 65,536 tiles) called
    as the reference's QuantizedLinear calls it (chunk_size=8): one launch per
    direction here, against the same call with chunk_size=None.  And the
    node-only swap: the reference's own chunk loop (chunks of 8 tiles, each
    under an activation checkpoint, src/bcjr/bcjr_quant.py:85-122) calling this
    node, timed on 1,024 tiles and scaled to the tensor (extrapolated)."""
    from torch.utils.checkpoint import checkpoint
    from bcjr import bcjr_forward_backward, bcjr_quantize_weight, make_sign_vector
    cb = bcjr.make_3inst_codebook(16, dev)
    W0 = torch.randn(8192, 2048, device=dev, generator=torch.Generator(dev).manual_seed(6))
    G = torch.randn(8192, 2048, device=dev, generator=torch.Generator(dev).manual_seed(7))
    sl = torch.tensor(make_sign_vector(8192, 1), device=dev)
    sr = torch.tensor(make_sign_vector(2048, 2), device=dev)
    out = {}
    for name, ch in (("chunk_size_8", 8), ("chunk_size_none", None)):
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        W = W0.clone().requires_grad_(True)
        bcjr_quantize_weight(W, sl, sr, cb, T, chunk_size=ch, L=16, k=2, V=1).backward(G)
        torch.cuda.synchronize(dev)
        out[name + "_s"] = time.perf_counter() - t0
    seqs = torch.randn(1024, 256, 1, device=dev, generator=torch.Generator(dev).manual_seed(8)).requires_grad_(True)
    gs = torch.randn_like(seqs)

    def chunk(s):
        return bcjr_forward_backward(s, cb, T, L=16, k=2, V=1)[0]

    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    soft = torch.cat([checkpoint(chunk, seqs[i:i + 8], use_reentrant=False) for i in range(0, 1024, 8)])
    soft.backward(gs)
    torch.cuda.synchronize(dev)
    node_only = time.perf_counter() - t0
    out["node_only_swap_s_extrapolated"] = node_only * 65536 / 1024
    out["note"] = ("gate tensor, 65,536 tiles, fwd + bwd: bcjr_quantize_weight ignores chunk_size (one launch per "
                   "direction); node_only_swap: the reference's chunk loop of 8 tiles per node call with activation "
                   "checkpointing, measured on 1,024 tiles and scaled x64")
    return out


def dequant_layer(torch, bcjr, ops, dev):
    """Dequantization of a Llama-3.2-1B decoder layer from the packed 2-bit format
    (HYB L=16, k=2, V=2): bcjr_dequant per tensor (walk replay + codebook +
    untiling + scale into the rotated-basis matrix) and the inverse RHT after it.
    Algorithmic bytes of bcjr_dequant per weight: a 4-byte write plus 2 bits of
    packed bitstream; the kernel is HBM-bound."""
    import numpy as np
    lut = np.random.default_rng(5).standard_normal((512, 2)).astype(np.float32)
    cb = bcjr.make_hyb_codebook_gpu(lut, 9, 16, dev)
    spec = ops.Spec(16, 2, 2, ops.CODE_HYB, 9)
    stream = torch.cuda.current_stream(dev)
    tot_k = tot_r = 0.0
    per = {}
    for name, rows, cols, _ in LAYER_TENSORS:
        B = rows * cols // 256
        g = torch.Generator(dev).manual_seed(rows + cols)
        packed = torch.randint(0, 256, (B, 64), dtype=torch.uint8, device=dev, generator=g)
        start = torch.randint(0, 1 << 16, (B,), dtype=torch.int32, device=dev, generator=g)
        sl = torch.ones(rows, device=dev)
        sr = torch.ones(cols, device=dev)
        W = ops.dequant(spec, start, cb._bcjr_lut, rows, cols, 16, 16, 0.02, packed=packed)
        bcjr.apply_inverse_rht_gpu(W, sl, sr)
        e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        # A few ms of spin ahead of the events, so the host has enqueued both
        # launches before the first event fires: the events then bracket the
        # kernels alone, not the host's enqueue gap (longer than a 4 M-weight
        # dequant).
        torch.cuda._sleep(5_000_000)
        e[0].record(stream)
        W = ops.dequant(spec, start, cb._bcjr_lut, rows, cols, 16, 16, 0.02, packed=packed)
        e[1].record(stream)
        bcjr.apply_inverse_rht_gpu(W, sl, sr)
        e[2].record(stream)
        torch.cuda.synchronize(dev)
        kd, kr = e[0].elapsed_time(e[1]) / 1e3, e[1].elapsed_time(e[2]) / 1e3
        per[name] = {"dequant_us": kd * 1e6, "GB_s": rows * cols * 4.25 / kd / 1e9}
        tot_k += kd
        tot_r += kr
    big = max(LAYER_TENSORS, key=lambda t: t[1] * t[2])
    return {"layer_seconds": tot_k + tot_r, "dequant_seconds": tot_k, "inverse_rht_seconds": tot_r,
            "roofline": {"bound": "hbm", "kernel": "bcjr_dequant_t16_kernel<4,2,HYB,packed>", "tensor": big[0],
                         "achieved": per[big[0]]["GB_s"], "peak": 8000.0, "unit": "GB/s",
                         "frac": per[big[0]]["GB_s"] / 8000.0, "bytes_per_weight": 4.25},
            "tensors": per}


def experts_leg(torch, bcjr, dev, E, T=0.1):
    """Expert-batched dispatch on OLMoE-1B-7B expert shapes (gate 1024x2048, up
    1024x2048, down 2048x1024 per expert; N(0,1) weights times a lognormal
    (sigma 0.5) scale per expert; L=16, k=2, V=1, 3INST): E experts' 3E weights
    soft-quantized forward + backward in one bcjr_quantize_experts call, against
    one bcjr_quantize_weight per weight (the reference's per-expert loop)."""
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

    def batched():
        lat = [w.detach().requires_grad_(True) for w in Ws]
        torch.autograd.backward(bcjr.bcjr_quantize_experts(lat, sl, sr, cb, T, **kw), gs)

    def loop():
        lat = [w.detach().requires_grad_(True) for w in Ws]
        for w, a, b, gg in zip(lat, sl, sr, gs):
            bcjr.bcjr_quantize_weight(w, a, b, cb, T, **kw).backward(gg)

    res = {}
    for name, fn in (("batched", batched), ("loop", loop)):
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize(dev)
        res[name] = time.perf_counter() - t0
    seqs = sum(r * c // 256 for r, c in shapes)
    out = {"experts": E, "weights": 3 * E, "sequences": seqs, "batched_seconds": res["batched"],
           "loop_seconds": res["loop"], "state_updates_per_s": 4.0 * seqs * 256 * 65536 / res["batched"],
           "note": "OLMoE-1B-7B expert shapes, lognormal per-expert scales, 3INST L=16 k=2 V=1, T=%g, fwd + bwd "
                   "including both RHTs" % T}
    if E >= 64:
        out["layer_64_experts_seconds"] = res["batched"] * 64 / E  # measured whole
    else:
        out["layer_64_experts_seconds_extrapolated"] = res["batched"] * 64 / E
        out["note"] += "; the 64-expert figure is the %d-expert time scaled by 64/%d" % (E, E)
    return out


def calibration_copy(torch, dev):
    """One device-to-device copy of CALIB_BYTES: its FETCH_SIZE / WRITE_SIZE
    counters scale the BCJR kernels' counters to bytes."""
    src = torch.ones(CALIB_BYTES // 4, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize(dev)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the path shards across GPUs by "
              "tiles with no collective inside BCJR.", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch
    import bcjr
    from bcjr import ops

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    peaks = measure_peaks(torch, dev)
    exp_peak = peaks["exp"]["per_s"]

    if args.config == "cpu":  # the CPU-runnable config on the GPU (a latency figure: 128 sequences)
        L, N, B = 12, 256, 128
        cb = bcjr.make_1mad_codebook(L, dev)
        x = torch.tensor(np.random.default_rng(0).standard_normal((B, N, 1)).astype(np.float32), device=dev)
        g = torch.tensor(np.random.default_rng(1).standard_normal((B, N, 1)).astype(np.float32), device=dev)

        def step():
            xs = x.detach().requires_grad_(True)
            bcjr.bcjr_forward_backward(xs, cb, 0.1, L=L, k=2, V=1)[0].backward(g)

        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize(dev)
        sec = (time.perf_counter() - t0) / args.steps
        print(json.dumps({"metric": METRIC, "value": 4.0 * B * N * (1 << L) / sec, "unit": "state-updates/s",
                          "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": sec * 1e3,
                          "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
                          "data": "synthetic N(0,1) (seed 0), upstream gradient N(0,1) (seed 1)",
                          "config": {"workload": "cpu-config: L=12 k=2 V=1 N=256 B=128, 1MAD, T=0.1"}}),
              flush=True)
        return

    if args.config == "tile":
        res = tile_config(torch, bcjr, ops, dev, exp_peak)
        calibration_copy(torch, dev)
        print(json.dumps({"metric": METRIC, "value": res["state_updates_per_s"], "unit": "state-updates/s",
                          "n_gpus": 1, "steps": 3, "warmup": 1, "ms_per_step": res["fwd_ms"] + res["bwd_ms"],
                          "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
                          "data": "synthetic N(0,1)", "config": {"workload": res["workload"]}, "tile": res}),
              flush=True)
        return

    if args.config in ("qat", "qat_layer", "dequant"):  # one secondary leg alone, for the profiler
        leg = {"qat": qat_shape, "qat_layer": qat_layer}.get(args.config)
        res = leg(torch, bcjr, ops, dev, exp_peak) if leg else dequant_layer(torch, bcjr, ops, dev)
        calibration_copy(torch, dev)
        print(json.dumps({"config": args.config, args.config: res}), flush=True)
        return

    progress("layer: building the seven weights")
    layer = Layer(torch, bcjr, dev)
    cells = float(LAYER_SEQS) * 256 * 65536
    stream = torch.cuda.current_stream(dev)

    # ---- the layer QAT step, timed whole ----
    ms_step = None
    if not args.kernels_only:
        for _ in range(args.warmup):
            layer.step()
        torch.cuda.synchronize(dev)
        progress(f"layer: {args.warmup} warmup step(s) done")
        t0 = time.perf_counter()
        for _ in range(args.steps):
            layer.step()
        torch.cuda.synchronize(dev)
        ms_step = (time.perf_counter() - t0) / args.steps * 1e3
        progress(f"layer: {args.steps} timed step(s), {ms_step:.1f} ms per step")

    # ---- the step's three launches, one at a time ----
    fwd_s, bwd_s, vit_s = layer_kernels(torch, ops, layer, dev)
    soft_s = fwd_s + bwd_s
    per_cell = trans_per_cell_grad(2)
    traffic = read_traffic()
    roofline = {"bound": "valu_exp", "kernel": "bcjr_fwd4_kernel<2,4> + bcjr_bwd_kernel<2,1,2,8,6,8> (the layer's soft launches)",
                "achieved": per_cell * cells / soft_s / 1e12, "peak": exp_peak / 1e12, "unit": "Texp/s",
                "frac": per_cell * cells / soft_s / exp_peak, "traffic": traffic,
                "per_cell": per_cell, "cells": cells, "launch_s": soft_s,
                "exp_floor_s": per_cell * cells / exp_peak}
    if traffic is not None:
        roofline["hbm_GB_s"] = traffic / soft_s / 1e9
        roofline["hbm_floor_s"] = traffic / 8e12
        roofline["hbm_frac"] = traffic / soft_s / 8e12
    kernels = {
        "bcjr_fwd4_kernel": {"s": fwd_s, "trans_per_cell": trans_per_cell_soft(2),
                            "frac": trans_per_cell_soft(2) * cells / fwd_s / exp_peak},
        "bcjr_bwd_kernel": {"s": bwd_s, "trans_per_cell": 2.0, "frac": 2.0 * cells / bwd_s / exp_peak},
        "bcjr_viterbi_kernel": {"s": vit_s, "cell_updates_per_s": cells / vit_s},
    }
    step_s = ms_step / 1e3 if ms_step is not None else fwd_s + bwd_s + vit_s
    line = {
        "metric": METRIC, "value": 4.0 * cells / step_s, "unit": "state-updates/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": step_s * 1e3, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: N(0,1) latent weights (seed 0) and upstream gradients (seed 1), random sign vectors",
        "config": {"workload": "Llama-3.2-1B decoder-layer QAT step: q/o 2048x2048, k/v 512x2048, gate/up "
                               "8192x2048, down 2048x8192 (237,568 tiles of 256), L=16 k=2 V=1, 3INST, per-tensor "
                               "T q .05 k .08 v .12 o .2 gate .3 up .4 down .5; RHT + soft fwd + bwd (one launch "
                               "each) + Viterbi 2-bit pack",
                   "tiles": LAYER_SEQS, "L": 16, "k": 2, "V": 1, "N": 256, "code": "3inst"},
        "layer_step_s": step_s,
        "roofline": roofline, "kernels": kernels,
        "peaks_per_s": {k_: v["per_s"] for k_, v in peaks.items()},
    }
    progress("layer: per-kernel launches done")
    if not args.no_secondary:
        legs = (("tile", lambda: tile_config(torch, bcjr, ops, dev, exp_peak)),
                ("qat_shape", lambda: qat_shape(torch, bcjr, ops, dev, exp_peak)),
                ("qat_layer", lambda: qat_layer(torch, bcjr, ops, dev, exp_peak)),
                ("drop_in", lambda: drop_in_chunked(torch, bcjr, dev)),
                ("dequant", lambda: dequant_layer(torch, bcjr, ops, dev)))
        if args.experts > 0:
            legs += (("experts", lambda: experts_leg(torch, bcjr, dev, args.experts)),)
        line["secondary"] = {}
        for name, leg in legs:
            line["secondary"][name] = leg()
            progress(f"secondary {name} done")
    calibration_copy(torch, dev)
    if not args.no_cpu_baseline:
        x = layer.tiles()
        firsts = np.cumsum([0] + [r * c // 256 for _, r, c, _ in LAYER_TENSORS])[:7]
        rows = torch.tensor(firsts, device=dev)
        tiles_np = x[rows].cpu().numpy()
        tiles_T = layer.T_tiles[rows].cpu().numpy()
        tiles_g = np.random.default_rng(1).standard_normal(tiles_np.shape).astype(np.float32)
        del x
        progress("cpu baseline")
        line["cpu_baseline"] = cpu_baseline(args, tiles_np, tiles_T, tiles_g)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
