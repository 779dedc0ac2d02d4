"""On-disk format of quantized weights and their dequantization on gfx950.

Drop-in for src/quantize/serialize.py:18-107 and precompute_walk_states
(src/quantize/lut_ft.py:59-79):

  * save_quantized writes the reference's payload unchanged (a torch.save'd dict
    of numpy arrays: bitstreams (n_col_blocks, n_row_blocks, n_steps) uint8 with
    one step per byte, start_states int32, int8 sign vectors, W_scale, shape,
    meta, config), so the reference's load_quantized reads these files and
    load_quantized here reads the reference's.
  * load_quantized opens them with torch.load(weights_only=True), allowlisting
    only numpy's array reconstruction, so nothing in the file is executed.
  * save_packed / load_packed: the packed format, a safetensors file holding
    the bitstream at k*V bits per step (2 bits per weight for k = 2; the
    reference's one-step-per-byte layout spends 8 / (k*V) times that), LSB-first
    within each byte, step t of a tile in bits [t*kV, (t+1)*kV) of its row, plus
    the same fields as the payload (W_scale as float64, config/meta as JSON).
  * dequant_target / dequant_target_gpu: walk replay, codebook lookup, untiling
    and scaling in one kernel (bcjr_dequant, every element decoded from the last
    ceil(L/kV) steps of its tile), then the inverse RHT on the FWHT kernels.
  * precompute_walk_states: the walks on the decode kernel.

Tiles follow the reference (src/quantize/blockldlq.py:74-110): tile (j, i) is
W[i*Tx:(i+1)*Tx, j*Ty:(j+1)*Ty] flattened row-major, step t holding elements
t*V .. t*V+V-1.
"""
from __future__ import annotations

import json
import os

import numpy as np
import torch

from . import ops
from .codes import resolve_codebook
from .ops import CODE_HYB, CODE_TABLE, Spec
from .rht import apply_inverse_rht_gpu

DEFAULT_CONFIG = {"L": 16, "k": 2, "V": 2, "Tx": 16, "Ty": 16}
PACKED_FORMAT = "bcjr-packed-v1"


def _np(x, dtype=None):
    if isinstance(x, torch.Tensor):
        x = x.detach().cpu().numpy()
    return np.asarray(x) if dtype is None else np.asarray(x, dtype=dtype)


# ---------------------------------------------------------------------------
# The reference's payload
# ---------------------------------------------------------------------------
def save_quantized(path, bitstreams, start_states, sign_l, sign_r, W_scale, shape, meta, config=None):
    """Write one quantized target in the reference's format (serialize.py:18-47).

    bitstreams (n_col_blocks, n_row_blocks, n_steps) values < 2^(k*V);
    start_states (n_col_blocks, n_row_blocks); sign vectors (m,), (n,) of +-1."""
    if config is None:
        config = dict(DEFAULT_CONFIG)
    payload = {
        "bitstreams": np.ascontiguousarray(_np(bitstreams), dtype=np.uint8),
        "start_states": np.ascontiguousarray(_np(start_states), dtype=np.int32),
        "sign_l": np.sign(_np(sign_l)).astype(np.int8),
        "sign_r": np.sign(_np(sign_r)).astype(np.int8),
        "W_scale": float(W_scale),
        "shape": tuple(int(d) for d in shape),
        "meta": meta,
        "config": config,
    }
    d = os.path.dirname(path)
    if d:
        os.makedirs(d, exist_ok=True)
    torch.save(payload, path)


def _numpy_array_globals():
    """The globals a pickled numpy array needs and nothing else: ndarray, dtype,
    the array reconstructor (under its numpy 1 and numpy 2 module paths) and the
    dtype classes of the payload's numeric types."""
    try:
        from numpy._core.multiarray import _reconstruct
    except ImportError:  # numpy 1.x
        from numpy.core.multiarray import _reconstruct
    names = [np.ndarray, np.dtype, _reconstruct,
             (_reconstruct, "numpy.core.multiarray._reconstruct"),
             (_reconstruct, "numpy._core.multiarray._reconstruct")]
    for t in (np.bool_, np.int8, np.uint8, np.int16, np.uint16, np.int32, np.uint32, np.int64, np.uint64,
              np.float16, np.float32, np.float64):
        names.append(type(np.dtype(t)))
    return names


def load_quantized(path):
    """Payload dict of a saved target (serialize.py:50-52).  Reads the
    reference's .pt payloads with torch.load(weights_only=True) and numpy's
    array reconstruction allowlisted, so loading executes nothing from the
    file; .safetensors files go through load_packed."""
    if str(path).endswith(".safetensors"):
        return load_packed(path)
    with torch.serialization.safe_globals(_numpy_array_globals()):
        return torch.load(path, weights_only=True, map_location="cpu")


# ---------------------------------------------------------------------------
# Packed format
# ---------------------------------------------------------------------------
def _check_kv(kV):
    if kV not in (1, 2, 4, 8):
        raise AssertionError(f"packing needs k*V in (1, 2, 4, 8); got {kV}")


def pack_bitstreams(bitstreams, kV):
    """(..., n_steps) step indices -> (..., ceil(n_steps*kV/8)) uint8, LSB-first."""
    _check_kv(kV)
    b = _np(bitstreams).astype(np.uint8) & np.uint8((1 << kV) - 1)
    per = 8 // kV
    n_steps = b.shape[-1]
    pad = (-n_steps) % per
    if pad:
        b = np.concatenate([b, np.zeros(b.shape[:-1] + (pad,), np.uint8)], axis=-1)
    b = b.reshape(b.shape[:-1] + (-1, per))
    shifts = (np.arange(per, dtype=np.uint8) * kV).astype(np.uint8)
    return np.bitwise_or.reduce(b << shifts, axis=-1).astype(np.uint8)


def unpack_bitstreams(packed, n_steps, kV):
    """Inverse of pack_bitstreams: (..., n_steps) uint8 step indices."""
    _check_kv(kV)
    p = _np(packed).astype(np.uint8)
    per = 8 // kV
    t = np.arange(n_steps)
    return ((p[..., t // per] >> ((t % per) * kV).astype(np.uint8)) & np.uint8((1 << kV) - 1)).astype(np.uint8)


def save_packed(path, bitstreams, start_states, sign_l, sign_r, W_scale, shape, meta, config=None):
    """Write one target in the packed safetensors format; same arguments as
    save_quantized."""
    from safetensors.numpy import save_file

    if config is None:
        config = dict(DEFAULT_CONFIG)
    kV = int(config["k"]) * int(config["V"])
    bits = _np(bitstreams)
    tensors = {
        "packed": np.ascontiguousarray(pack_bitstreams(bits, kV)),
        "start_states": np.ascontiguousarray(_np(start_states), dtype=np.int32),
        "sign_l": np.sign(_np(sign_l)).astype(np.int8),
        "sign_r": np.sign(_np(sign_r)).astype(np.int8),
        "W_scale": np.asarray(float(W_scale), dtype=np.float64),
    }
    metadata = {
        "format": PACKED_FORMAT,
        "n_steps": str(int(bits.shape[-1])),
        "shape": json.dumps([int(d) for d in shape]),
        "config": json.dumps(config),
        "meta": json.dumps(meta),
    }
    d = os.path.dirname(path)
    if d:
        os.makedirs(d, exist_ok=True)
    save_file(tensors, path, metadata=metadata)


def load_packed(path):
    """Payload dict of a packed file: the keys of load_quantized with
    "packed" (n_col_blocks, n_row_blocks, ceil(n_steps*kV/8)) uint8 and
    "n_steps" in place of "bitstreams"."""
    from safetensors import safe_open

    with safe_open(path, framework="numpy") as f:
        md = f.metadata() or {}
        if md.get("format") != PACKED_FORMAT:
            raise ValueError(f"{path}: not a {PACKED_FORMAT} file (format={md.get('format')!r})")
        t = {k: f.get_tensor(k) for k in f.keys()}
    return {
        "packed": t["packed"],
        "n_steps": int(md["n_steps"]),
        "start_states": t["start_states"],
        "sign_l": t["sign_l"],
        "sign_r": t["sign_r"],
        "W_scale": float(t["W_scale"]),
        "shape": tuple(json.loads(md["shape"])),
        "meta": json.loads(md["meta"]),
        "config": json.loads(md["config"]),
    }


def bitstreams_of(saved):
    """(n_col_blocks, n_row_blocks, n_steps) uint8 of either payload kind."""
    if "bitstreams" in saved:
        return _np(saved["bitstreams"])
    cfg = saved["config"]
    return unpack_bitstreams(saved["packed"], saved["n_steps"], int(cfg["k"]) * int(cfg["V"]))


# ---------------------------------------------------------------------------
# Dequantization on the GPU
# ---------------------------------------------------------------------------
def _codebook_source(L, k, V, codebook=None, decode_fn=None, device="cuda"):
    """Spec and kernel table pointer source for a codebook tensor (tagged by
    the generators of .codes, or a plain (2^L, V) table) or a reference-style
    decode_fn (uint32 states -> (2^L,) or (2^L, V)), as precompute_codebook_v
    (src/viterbi/encode.py:233-247) materialises it."""
    if codebook is None:
        if decode_fn is None:
            raise AssertionError("dequant needs a codebook tensor or a decode_fn")
        res = np.asarray(decode_fn(np.arange(1 << L, dtype=np.uint32)))
        if res.ndim == 1:
            res = res[:, None]
        if res.shape != (1 << L, V):
            raise AssertionError(f"decode_fn returned shape {res.shape}, expected {(1 << L, V)}")
        codebook = torch.from_numpy(np.ascontiguousarray(res, dtype=np.float32)).to(device)
    return resolve_codebook(codebook, L, k, V, torch.device(device))


def dequant_target_gpu(saved, codebook=None, decode_fn=None, device="cuda", rotated=False):
    """Dequantized weight (m, n) float32 on `device` from a payload of either
    kind (src/quantize/serialize.py:55-107 dequant_target, on the GPU).  rotated=True stops before the inverse RHT (the rotated-basis matrix
    W_unit * W_scale that in-place QAT trains)."""
    device = torch.device(device)
    cfg = saved["config"]
    L, k, V, Tx, Ty = (int(cfg[x]) for x in ("L", "k", "V", "Tx", "Ty"))
    m, n = (int(d) for d in saved["shape"])
    n_col, n_row = n // Ty, m // Tx
    if m % Tx or n % Ty:
        raise AssertionError(f"shape {(m, n)} is not a whole number of {Tx}x{Ty} tiles")
    start = torch.from_numpy(np.ascontiguousarray(_np(saved["start_states"]), dtype=np.int32)).to(device)
    if tuple(start.shape) != (n_col, n_row):
        raise AssertionError(f"start_states {tuple(start.shape)} != {(n_col, n_row)}")
    spec, table = _codebook_source(L, k, V, codebook, decode_fn, device)
    if "bitstreams" in saved:
        bits = torch.from_numpy(np.ascontiguousarray(_np(saved["bitstreams"]), dtype=np.uint8)).to(device)
        if tuple(bits.shape) != (n_col, n_row, (Tx * Ty) // V):
            raise AssertionError(f"bitstreams {tuple(bits.shape)} != {(n_col, n_row, (Tx * Ty) // V)}")
        W = ops.dequant(spec, start, table, m, n, Tx, Ty, float(saved["W_scale"]), bitstream=bits)
    else:
        if int(saved["n_steps"]) != (Tx * Ty) // V:
            raise AssertionError(f"n_steps {saved['n_steps']} != {(Tx * Ty) // V}")
        packed = torch.from_numpy(np.ascontiguousarray(_np(saved["packed"]), dtype=np.uint8)).to(device)
        W = ops.dequant(spec, start, table, m, n, Tx, Ty, float(saved["W_scale"]), packed=packed)
    if rotated:
        return W
    sl = torch.from_numpy(_np(saved["sign_l"]).astype(np.float32)).to(device)
    sr = torch.from_numpy(_np(saved["sign_r"]).astype(np.float32)).to(device)
    return apply_inverse_rht_gpu(W, sl, sr)


def dequant_target(saved, decode_fn=None, codebook=None, device="cuda"):
    """Reconstruct the dequantized weight (serialize.py:56-107): (m, n) float64
    numpy array, computed on the GPU.  decode_fn is the reference's codebook
    callable; a codebook tensor (e.g. make_hyb_codebook_gpu) may be passed
    instead and is hashed in-kernel."""
    return dequant_target_gpu(saved, codebook=codebook, decode_fn=decode_fn, device=device).cpu().numpy() \
        .astype(np.float64)


def precompute_walk_states(bitstreams, start_states, L_bits=16, kV=4, device="cuda", as_tensor=False):
    """State walks (n_col_blocks, n_row_blocks, n_steps) int64 (lut_ft.py:59-79),
    replayed on the decode kernel.  Returns numpy unless as_tensor=True (then an
    int64 tensor on `device`)."""
    device = torch.device(device)
    bits = torch.from_numpy(np.ascontiguousarray(_np(bitstreams), dtype=np.int32)).to(device)
    start = torch.from_numpy(np.ascontiguousarray(_np(start_states), dtype=np.int32)).to(device)
    shape = tuple(bits.shape)
    B = int(np.prod(shape[:-1]))
    if tuple(start.shape) != shape[:-1]:
        raise AssertionError(f"start_states {tuple(start.shape)} != {shape[:-1]}")
    spec = Spec(L_bits, kV, 1, CODE_TABLE)
    walk = ops.decode_walks(spec, start.reshape(B), bits.reshape(B, shape[-1])).reshape(shape).to(torch.int64)
    return walk if as_tensor else walk.cpu().numpy()


__all__ = ["DEFAULT_CONFIG", "PACKED_FORMAT", "save_quantized", "load_quantized", "pack_bitstreams",
           "unpack_bitstreams", "save_packed", "load_packed", "bitstreams_of", "dequant_target",
           "dequant_target_gpu", "precompute_walk_states"]
