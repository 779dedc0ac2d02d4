"""GPU parity on the workloads the throughput figures are quoted on.

Every test runs the production launch shape (the whole batch in one forward,
one backward and one Viterbi launch) and checks:
  * chosen sequences against the float64 oracle: soft (max-norm relative
    1e-4), log Z (1e-5 relative), gradient (1e-3), and a bit-exact Viterbi
    (walk, bitstream, start state, reconstruction, 2-bit pack);
  * every sequence through size-independent properties: finite outputs, soft
    codewords inside the codebook's range (a soft codeword is a convex
    combination of codewords), the packed bitstream unpacking to the
    bitstream, the reconstruction equal to the codebook at the walk.

Workloads (L=16, k=2, V=1, 3INST, 256 weights per sequence):
  * the Llama-3.2-1B decoder layer: q/o 2048x2048, k/v 512x2048, gate/up
    8192x2048, down 2048x8192 (237,568 sequences), per-tensor T q .05, k .08,
    v .12, o .2, gate .3, up .4, down .5, fwd + bwd + Viterbi pack;
  * the same kernel instance at a batch of 4 grid-strides per workgroup, T
    alternating across the exact / group-sum variants within each workgroup;
  * the MLP block (gate/up/down at full shape, per-row lognormal scales)
    through bcjr_quantize_weight (RHT, RMS scale, tiles, node, inverse RHT);
  * the OLMoE-1B-7B MoE layer whole: 64 experts (gate/up 1024x2048, down
    2048x1024, lognormal per-expert scales, T = 0.1, 1,572,864 sequences)
    through one bcjr_quantize_experts call.
"""
import ctypes
import sys

import numpy as np
import pytest
import torch

from conftest import max_rel

pytestmark = pytest.mark.gpu

SOFT_TOL, GRAD_TOL, LOGZ_TOL = 1e-4, 1e-3, 1e-5
L, K, V, N = 16, 2, 1, 256
LAYER_TENSORS = (("q", 2048, 2048, 0.05), ("k", 512, 2048, 0.08), ("v", 512, 2048, 0.12),
                 ("o", 2048, 2048, 0.2), ("gate", 8192, 2048, 0.3), ("up", 8192, 2048, 0.4),
                 ("down", 2048, 8192, 0.5))


def _say(msg):
    print(f"[gpu-configs] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def cb3(bcjr_mod):
    cb = bcjr_mod.make_3inst_codebook(L, "cuda")
    return cb, cb.cpu().numpy()


def _check_against_oracle(oracle, seq_np, g_np, T_np, idx, dev_out, cb_np, what):
    """Oracle parity of the sequences `idx`.  dev_out maps soft, logZ, grad (or
    None) and the Viterbi outputs to device tensors over the whole batch; only
    the chosen rows are copied back."""
    rows = torch.tensor(idx, device="cuda")
    h = {k_: (None if v is None else v[rows].cpu().numpy()) for k_, v in dev_out.items()}
    for j, b in enumerate(idx):
        s1 = seq_np[b:b + 1]
        T = float(T_np[b])
        s_ref, z_ref = oracle.bcjr_forward(s1, cb_np, T, L, K * V)
        r_soft = max_rel(h["soft"][j:j + 1], s_ref)
        r_z = abs(float(h["logZ"][j]) - float(z_ref[0])) / abs(float(z_ref[0]))
        assert r_soft < SOFT_TOL, f"{what} seq {b} T={T}: soft rel {r_soft:.2e}"
        assert r_z < LOGZ_TOL, f"{what} seq {b} T={T}: logZ rel {r_z:.2e}"
        if h.get("grad") is not None:
            d_ref = oracle.bcjr_backward(s1, cb_np, T, L, K * V, g_np[b:b + 1])
            r_g = max_rel(h["grad"][j:j + 1], d_ref)
            assert r_g < GRAD_TOL, f"{what} seq {b} T={T}: grad rel {r_g:.2e}"
        if h.get("walk") is not None:
            walk_r, bits_r, start_r, recon_r, _ = oracle.viterbi(s1, cb_np, L, K * V)
            assert (h["walk"][j] == walk_r[0]).all(), f"{what} seq {b}: walk"
            assert (h["bitstream"][j] == bits_r[0]).all(), f"{what} seq {b}: bitstream"
            assert int(h["start"][j]) == int(start_r[0]), f"{what} seq {b}: start"
            assert (h["recon"][j] == recon_r[0]).all(), f"{what} seq {b}: recon"
            assert (h["packed"][j] == oracle.pack_bits(bits_r, K * V)[0]).all(), f"{what} seq {b}: packed"


def _check_properties(soft, logZ, grad, vit, cb, what):
    """Size-independent properties over every sequence (device tensors)."""
    lo, hi = float(cb.min()), float(cb.max())
    assert torch.isfinite(soft).all() and torch.isfinite(logZ).all(), what
    # sum_s P = 1 up to float32 rounding, so the hull holds to the soft tolerance
    slack = SOFT_TOL * max(abs(lo), abs(hi))
    assert float(soft.min()) >= lo - slack and float(soft.max()) <= hi + slack, what
    if grad is not None:
        assert torch.isfinite(grad).all(), what
    if vit is not None:
        walk, bits = vit["walk"], vit["bitstream"]
        assert int(walk.min()) >= 0 and int(walk.max()) < (1 << L), what
        assert torch.equal(bits, walk & ((1 << (K * V)) - 1)), what
        # consecutive states share L - kV bits: walk_t = (walk_{t-1} << kV | bits_t) mod 2^L
        assert torch.equal(walk[:, 1:], ((walk[:, :-1] << (K * V)) | bits[:, 1:]) & ((1 << L) - 1)), what
        assert torch.equal(vit["recon"][:, :, 0], cb[walk.long(), 0]), what
        pk = vit["packed"].to(torch.int32)
        shifts = torch.arange(4, device=pk.device, dtype=torch.int32) * 2
        unpacked = ((pk.unsqueeze(-1) >> shifts) & 3).reshape(pk.shape[0], -1)[:, :N]
        assert torch.equal(unpacked, bits), what


def _max_blocks(bcjr_mod, op, B):
    """Workgroups resident at once for this problem (slots the workspace holds)."""
    from bcjr import _lib
    lib = _lib.load()
    big = _lib.Problem(L, K, V, B, N, _lib.CODE_3INST, 9, 1)
    one = _lib.Problem(L, K, V, 1, N, _lib.CODE_3INST, 9, 1)
    nb, n1 = ctypes.c_size_t(0), ctypes.c_size_t(0)
    _lib.check(lib.bcjr_workspace_bytes(ctypes.byref(big), op, ctypes.byref(nb)), "ws")
    _lib.check(lib.bcjr_workspace_bytes(ctypes.byref(one), op, ctypes.byref(n1)), "ws")
    return nb.value // n1.value


def test_layer_kernel_instance_slot_reuse_and_mixed_T(bcjr_mod, oracle, cb3):
    """The layer's kernel instance with every workgroup running 4 sequences in a
    row on its slot, T switching between the exact and group-sum variants from
    one sequence to the next (the backward switches at 0.08, the 1024-thread
    forward at 0.045)."""
    from bcjr import _lib, ops
    cb, cb_np = cb3
    G = min(_max_blocks(bcjr_mod, _lib.OP_FORWARD, 1 << 20), _max_blocks(bcjr_mod, _lib.OP_BACKWARD, 1 << 20))
    B = 4 * G + 16
    _say(f"layer instance: B={B} (resident workgroups {G})")
    TS = np.array([0.05, 0.3, 0.03, 0.12, 0.07, 0.5], dtype=np.float32)
    T_np = TS[(np.arange(B) // G) % len(TS)]
    seq = np.random.default_rng(0).standard_normal((B, N, V)).astype(np.float32)
    g = np.random.default_rng(1).standard_normal((B, N, V)).astype(np.float32)
    x, gg, Tt = torch.tensor(seq, device="cuda"), torch.tensor(g, device="cuda"), torch.tensor(T_np, device="cuda")
    spec, _ = bcjr_mod.codes.resolve_codebook(cb, L, K, V, torch.device("cuda"))
    soft, logZ = ops.forward(spec, x, Tt, None)
    grad = ops.backward(spec, x, Tt, None, gg)
    vit = ops.viterbi(spec, x, None)
    torch.cuda.synchronize()
    _check_properties(soft, logZ, grad, vit, cb, "layer instance")
    idx = sorted({0, 1, G - 1, G, 2 * G, 3 * G, 4 * G, 4 * G + 15, 2 * G + 7, 3 * G + G // 2})
    _check_against_oracle(oracle, seq, g, T_np, idx, dict(soft=soft, logZ=logZ, grad=grad, **vit), cb_np,
                          "layer instance")


def test_llama_layer_full(bcjr_mod, oracle, cb3):
    """One whole Llama-3.2-1B decoder-layer step as bench.py runs it: 237,568
    sequences in one forward and one backward launch with per-tensor T, then
    one Viterbi launch with the 2-bit pack."""
    from bcjr import ops
    cb, cb_np = cb3
    counts = [r * c // 256 for _, r, c, _ in LAYER_TENSORS]
    B = sum(counts)
    assert B == 237568
    _say(f"llama layer: B={B}")
    T_np = np.concatenate([np.full(n, T, dtype=np.float32) for n, (_, _, _, T) in zip(counts, LAYER_TENSORS)])
    seq = np.random.default_rng(0).standard_normal((B, N, V)).astype(np.float32)
    g = np.random.default_rng(1).standard_normal((B, N, V)).astype(np.float32)
    x, gg, Tt = torch.tensor(seq, device="cuda"), torch.tensor(g, device="cuda"), torch.tensor(T_np, device="cuda")
    spec, _ = bcjr_mod.codes.resolve_codebook(cb, L, K, V, torch.device("cuda"))
    soft, logZ = ops.forward(spec, x, Tt, None)
    grad = ops.backward(spec, x, Tt, None, gg)
    vit = ops.viterbi(spec, x, None)
    torch.cuda.synchronize()
    _say("llama layer: launches done")
    _check_properties(soft, logZ, grad, vit, cb, "llama layer")
    starts = np.cumsum([0] + counts)
    idx = sorted({int(i) for s0, s1 in zip(starts[:-1], starts[1:]) for i in (s0, s1 - 1)})
    _check_against_oracle(oracle, seq, g, T_np, idx, dict(soft=soft, logZ=logZ, grad=grad, **vit), cb_np,
                          "llama layer")


def _unit_tiles(bcjr_mod, Wrot):
    """RMS-normalised rotated weight as (B, N, 1) tiles and its scale, as
    bcjr_quantize_weight_rotated forms them (src/bcjr/bcjr_quant.py:135-150)."""
    from bcjr.quant import tile_for_viterbi
    scale = Wrot.pow(2).mean().sqrt().clamp(min=1e-30)
    seqs, _ = tile_for_viterbi(Wrot / scale)
    return seqs.unsqueeze(-1), scale


def _spot_check_weight(bcjr_mod, oracle, cb_np, W, sl, sr, Wq, Wgrad, G, T, nt, what):
    """Oracle parity of tiles `nt` of one weight quantized by bcjr_quantize_weight:
    the GPU's rotated tiles are the oracle's input; the GPU's soft tiles are
    read back through the (orthogonal) RHT of W_q; the gradient with respect to
    the tiles is the RHT of W.grad, times the scale, tiled."""
    from bcjr import apply_rht_gpu
    from bcjr.quant import tile_for_viterbi
    with torch.no_grad():
        seqs, scale = _unit_tiles(bcjr_mod, apply_rht_gpu(W, sl, sr))
        soft_t, _ = tile_for_viterbi(apply_rht_gpu(Wq, sl, sr) / scale)
        g_t, _ = tile_for_viterbi(apply_rht_gpu(G, sl, sr) * scale)
        d_t, _ = tile_for_viterbi(apply_rht_gpu(Wgrad, sl, sr) * scale)
    rows = torch.tensor(nt, device="cuda")
    s_np = seqs[rows].cpu().numpy()
    s_ref, _ = oracle.bcjr_forward(s_np, cb_np, T, L, K * V)
    # the RHT round trip adds float32 rounding (~1e-6 relative) on top of the node's error
    assert max_rel(soft_t[rows].cpu().numpy()[:, :, None], s_ref) < SOFT_TOL, f"{what}: soft"
    d_ref = oracle.bcjr_backward(s_np, cb_np, T, L, K * V, g_t[rows].cpu().numpy()[:, :, None])
    assert max_rel(d_t[rows].cpu().numpy()[:, :, None], d_ref) < GRAD_TOL, f"{what}: grad"
    assert torch.isfinite(Wq).all() and torch.isfinite(Wgrad).all(), what


def test_llama_mlp_block_full_shape(bcjr_mod, oracle, cb3):
    """gate/up 8192x2048 and down 2048x8192 weights, N(0,1) times a per-row
    lognormal scale (seed 0), through bcjr_quantize_weight at T = 0.1 with one
    backward each (196,608 sequences)."""
    from bcjr import bcjr_quantize_weight, make_sign_vector
    cb, cb_np = cb3
    rng = np.random.default_rng(0)
    for name, (m, n) in (("gate", (8192, 2048)), ("up", (8192, 2048)), ("down", (2048, 8192))):
        _say(f"mlp {name} {m}x{n}")
        W_np = rng.standard_normal((m, n)).astype(np.float32) * np.exp(0.5 * rng.standard_normal((m, 1))).astype(np.float32)
        W = torch.tensor(W_np, device="cuda", requires_grad=True)
        sl = torch.tensor(make_sign_vector(m, 1), device="cuda")
        sr = torch.tensor(make_sign_vector(n, 2), device="cuda")
        Wq = bcjr_quantize_weight(W, sl, sr, cb, 0.1, L=L, k=K, V=V)
        G = torch.randn(m, n, device="cuda", generator=torch.Generator("cuda").manual_seed(3))
        (Wq * G).sum().backward()
        B = m * n // 256
        _spot_check_weight(bcjr_mod, oracle, cb_np, W.detach(), sl, sr, Wq.detach(), W.grad, G, 0.1,
                           [0, B // 3, B - 1], f"mlp {name}")


def test_olmoe_64_experts_whole_layer(bcjr_mod, oracle, cb3):
    """The OLMoE-1B-7B MoE layer whole: 64 experts, each gate/up 1024x2048 and
    down 2048x1024 (192 weights, 402,653,184 weights, 1,572,864 sequences),
    N(0,1) weights times a lognormal (sigma 0.5, seed 0) per-expert scale, every
    weight in ONE bcjr_quantize_experts call at T = 0.1 (one forward and one
    backward launch over all 1,572,864 sequences), where the reference loops the
    experts (src/qat/qat_moe_layer.py:106-114).  Every output: finite, the
    gradient finite, and every soft tile (read back through the orthogonal RHT of
    W_q) inside the codebook's hull.  The first and last tile of seven weights
    (gate, up and down of the first, a middle and the last expert) against the
    oracle composition."""
    from bcjr import bcjr_quantize_experts, make_sign_vector
    from bcjr.quant import tile_for_viterbi
    from bcjr.rht import apply_rht_batched
    cb, cb_np = cb3
    E = 64
    rng = np.random.default_rng(0)
    scales = np.exp(0.5 * rng.standard_normal(E)).astype(np.float32)
    shapes = [(1024, 2048), (1024, 2048), (2048, 1024)] * E
    gen = torch.Generator("cuda").manual_seed(0)
    Ws = [(torch.randn(s, device="cuda", generator=gen) * float(scales[i // 3])).requires_grad_(True)
          for i, s in enumerate(shapes)]
    sl = [torch.tensor(make_sign_vector(s[0], 10 + i), device="cuda") for i, s in enumerate(shapes)]
    sr = [torch.tensor(make_sign_vector(s[1], 500 + i), device="cuda") for i, s in enumerate(shapes)]
    seqs = sum(m * n // 256 for m, n in shapes)
    assert seqs == 1572864
    _say(f"olmoe: {E} experts, {len(shapes)} weights, {seqs} sequences in one call")
    outs = bcjr_quantize_experts(Ws, sl, sr, cb, 0.1, L=L, k=K, V=V)
    Gs = [torch.randn(s, device="cuda", generator=gen) for s in shapes]
    torch.autograd.backward(outs, Gs)
    torch.cuda.synchronize()
    _say("olmoe: forward + backward done")
    lo, hi = float(cb.min()), float(cb.max())
    slack = 1e-4 * max(abs(lo), abs(hi))  # the RHT round trip adds float32 rounding
    with torch.no_grad():
        for shape in ((1024, 2048), (2048, 1024)):
            idx = [i for i, s in enumerate(shapes) if s == shape]
            for c0 in range(0, len(idx), 32):
                part = idx[c0:c0 + 32]
                Wq = torch.stack([outs[i] for i in part])
                assert torch.isfinite(Wq).all(), f"olmoe W_q {part[0]}..{part[-1]}"
                assert all(torch.isfinite(Ws[i].grad).all() for i in part), f"olmoe grad {part[0]}.."
                SL, SR = torch.stack([sl[i] for i in part]), torch.stack([sr[i] for i in part])
                Wt = apply_rht_batched(torch.stack([Ws[i].detach() for i in part]), SL, SR)
                scale = Wt.pow(2).mean(dim=(1, 2)).sqrt()
                soft_rot = apply_rht_batched(Wq, SL, SR) / scale[:, None, None]
                assert float(soft_rot.min()) >= lo - slack and float(soft_rot.max()) <= hi + slack, \
                    f"olmoe hull {part[0]}..{part[-1]}"
                del Wq, Wt, soft_rot
    for i in (0, 1, 2, 97, 188, 190, 191):
        B = shapes[i][0] * shapes[i][1] // 256
        _spot_check_weight(bcjr_mod, oracle, cb_np, Ws[i].detach(), sl[i], sr[i], outs[i].detach(), Ws[i].grad,
                           Gs[i], 0.1, [0, B - 1], f"olmoe weight {i}")
