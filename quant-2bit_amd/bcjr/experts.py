"""Expert-batched dispatch of the BCJR quantizer (mixture-of-experts layers).

The reference quantizes an OLMoE layer's experts one weight at a time: the
dispatch loop of QATMoELayer.forward (src/qat/qat_moe_layer.py:106-114) calls
each QATExpert, whose two QuantizedLinear modules each run
bcjr_quantize_weight (src/bcjr/bcjr_quant.py:159-178) -- 2 x num_experts
RHTs, BCJR calls and inverse RHTs per layer step.

bcjr_quantize_experts does the same arithmetic for any list of weights in
    one batched RHT launch pair per distinct shape,
    one BCJR forward (and one backward) for the tiles of every weight, with
        each weight's temperature carried per sequence,
    one batched inverse RHT per distinct shape,
so a whole layer's experts cost a single engine call.  Each weight keeps its
own detached RMS scale (bcjr_quant.py:140) and its own sign vectors, and the
result for every weight is that of bcjr_quantize_weight on it alone: every
sequence is computed independently of what else is in the batch.
"""
from __future__ import annotations

from collections import OrderedDict

import torch

from .forward_backward import K_BITS, L_BITS, V_DIM, bcjr_forward_backward
from .quant import TX, TY
from .rht import apply_inverse_rht_batched, apply_rht_batched
from .viterbi import viterbi_encode_v_batched_hip


def _per_weight_T(T_temps, E, device):
    """(E,) float32 temperatures from a float, a 0-d tensor or E values."""
    if torch.is_tensor(T_temps):
        t = T_temps.detach().to(device=device, dtype=torch.float32).reshape(-1)
    else:
        try:
            t = torch.tensor([float(x) for x in T_temps], dtype=torch.float32, device=device)
        except TypeError:
            t = torch.tensor([float(T_temps)], dtype=torch.float32, device=device)
    if t.numel() == 1:
        return t.expand(E)
    if t.numel() != E:
        raise AssertionError(f"T_temps has {t.numel()} values; expected 1 or {E}")
    return t


def bcjr_quantize_experts(W_latents, sign_l, sign_r, codebook, T_temps, Tx=TX, Ty=TY,
                          L=L_BITS, k=K_BITS, V=V_DIM):
    """Soft-quantize E weights in one engine call, in place of one
    bcjr_quantize_weight per expert weight (src/qat/qat_moe_layer.py:106-114 loops
    the experts).

    W_latents: sequence of E float32 GPU tensors (m_e, n_e) (gradients allowed),
               m_e, n_e powers of two divisible by Tx, Ty.
    sign_l, sign_r: sequences of E sign vectors (m_e,), (n_e,).
    T_temps: one temperature (float or 0-d tensor) or E of them.
    Returns the list of E quantized weights W_q (m_e, n_e), each differentiable
    with respect to its latent weight."""
    E = len(W_latents)
    if not (len(sign_l) == len(sign_r) == E):
        raise AssertionError(f"{E} weights but {len(sign_l)} / {len(sign_r)} sign vectors")
    if E == 0:
        return []
    device = W_latents[0].device
    T_w = _per_weight_T(T_temps, E, device)

    groups: "OrderedDict[tuple, list]" = OrderedDict()
    for e, W in enumerate(W_latents):
        if W.dim() != 2:
            raise AssertionError(f"weight {e} must be 2-D; got {tuple(W.shape)}")
        m, n = W.shape
        if m % Tx or n % Ty:
            raise AssertionError(f"weight {e} shape {(m, n)} not tileable by {(Tx, Ty)}")
        groups.setdefault((m, n), []).append(e)

    seqs, temps, meta = [], [], []
    for (m, n), idx in groups.items():
        G = len(idx)
        W = torch.stack([W_latents[e] for e in idx])
        SL = torch.stack([torch.as_tensor(sign_l[e], device=device, dtype=torch.float32) for e in idx])
        SR = torch.stack([torch.as_tensor(sign_r[e], device=device, dtype=torch.float32) for e in idx])
        Wt = apply_rht_batched(W, SL, SR)
        scale = Wt.detach().pow(2).mean(dim=(1, 2)).sqrt().clamp(min=1e-30)  # (G,)
        unit = Wt / scale[:, None, None]
        n_row, n_col = m // Tx, n // Ty
        # per weight, tile order col_block * n_row + row_block, 16x16 row-major
        s = unit.reshape(G, m, n_col, Ty).permute(0, 2, 1, 3).reshape(G * n_col * n_row, (Tx * Ty) // V, V)
        seqs.append(s)
        temps.append(T_w[idx].repeat_interleave(n_col * n_row))
        meta.append(((m, n), idx, SL, SR, scale, G * n_col * n_row))

    soft, _ = bcjr_forward_backward(torch.cat(seqs), codebook, torch.cat(temps), L=L, k=k, V=V)

    out = [None] * E
    for ((m, n), idx, SL, SR, scale, B), soft_g in zip(meta, torch.split(soft, [mm[-1] for mm in meta])):
        G = len(idx)
        n_col = n // Ty
        q_unit = soft_g.reshape(G, n_col, m, Ty).permute(0, 2, 1, 3).reshape(G, m, n)
        Wq = apply_inverse_rht_batched(q_unit * scale[:, None, None], SL, SR)
        for j, e in enumerate(idx):
            out[e] = Wq[j]
    return out


def ste_quantize_experts(W_latents, sign_l, sign_r, codebook, Tx=TX, Ty=TY, k=K_BITS):
    """Hard (T -> 0) quantization of E weights in one Viterbi launch: what
    quantize_forward_gpu (src/qat/ste.py:183-212) gives each weight, for a whole
    layer at once (QATMoELayer.prime_cache, src/qat/qat_moe_layer.py:129-135,
    loops experts instead).  No gradient: this primes caches and packs."""
    E = len(W_latents)
    if not (len(sign_l) == len(sign_r) == E):
        raise AssertionError(f"{E} weights but {len(sign_l)} / {len(sign_r)} sign vectors")
    if E == 0:
        return []
    S, V = codebook.shape
    L = int(S).bit_length() - 1
    device = W_latents[0].device
    groups: "OrderedDict[tuple, list]" = OrderedDict()
    for e, W in enumerate(W_latents):
        m, n = W.shape
        if m % Tx or n % Ty:
            raise AssertionError(f"weight {e} shape {(m, n)} not tileable by {(Tx, Ty)}")
        groups.setdefault((m, n), []).append(e)
    seqs, meta = [], []
    with torch.no_grad():
        for (m, n), idx in groups.items():
            G = len(idx)
            W = torch.stack([W_latents[e].detach().float() for e in idx])
            SL = torch.stack([torch.as_tensor(sign_l[e], device=device, dtype=torch.float32) for e in idx])
            SR = torch.stack([torch.as_tensor(sign_r[e], device=device, dtype=torch.float32) for e in idx])
            Wt = apply_rht_batched(W, SL, SR)
            scale = Wt.pow(2).mean(dim=(1, 2)).sqrt().clamp(min=1e-30)
            n_col = n // Ty
            s = (Wt / scale[:, None, None]).reshape(G, m, n_col, Ty).permute(0, 2, 1, 3).reshape(-1, Tx * Ty)
            seqs.append(s)
            meta.append(((m, n), idx, SL, SR, scale, s.shape[0]))
        _, _, recon, _ = viterbi_encode_v_batched_hip(torch.cat(seqs).contiguous(), codebook, L=L, k=k, V=V)
        out = [None] * E
        for ((m, n), idx, SL, SR, scale, B), rec in zip(meta, torch.split(recon, [mm[-1] for mm in meta])):
            G = len(idx)
            q = rec.reshape(G, n // Ty, m, Ty).permute(0, 2, 1, 3).reshape(G, m, n) * scale[:, None, None]
            Wq = apply_inverse_rht_batched(q, SL, SR)
            for j, e in enumerate(idx):
                out[e] = Wq[j]
    return out


def quantize_moe_experts(experts_weights, signs, codebook, T_temps, **kw):
    """Dict form for a layer: experts_weights maps a name (e.g. (expert, "gate_up"))
    to its latent weight, signs maps the same names to (sign_l, sign_r); returns a
    dict of quantized weights with the same names, from one engine call."""
    names = list(experts_weights)
    T = T_temps
    if isinstance(T_temps, dict):
        T = [float(T_temps[nm]) for nm in names]
    outs = bcjr_quantize_experts([experts_weights[nm] for nm in names], [signs[nm][0] for nm in names],
                                 [signs[nm][1] for nm in names], codebook, T, **kw)
    return dict(zip(names, outs))


__all__ = ["bcjr_quantize_experts", "ste_quantize_experts", "quantize_moe_experts"]
