"""CPU tests of the on-disk format (src/quantize/serialize.py:18-107) and the
oracle's dequantization (no GPU calls).

- the oracle's walk replay and dequantization, pinned by the C decode
  restatement, the sliding-window closed form of a state, a matrix assembled
  from tiles by slicing, and exact rational arithmetic for the scale;
- the reference payload: written and read back without executing anything,
  refused when it holds anything but numpy arrays and plain containers;
- the packed format: byte layout, round trips, 2 bits per weight;
- bcjr_dequant's argument validation without a device.
"""
import ctypes
import os
import pickle
from fractions import Fraction

import numpy as np
import pytest
import torch

import oracle as O


def _walk_closed_form(bits, start, L, KV):
    """s_t = (start * 2^(KV(t+1)) + sum_{tau<=t} b_tau 2^(KV(t-tau))) mod 2^L,
    in Python integers."""
    out = []
    for t in range(len(bits)):
        v = int(start) << (KV * (t + 1))
        for tau in range(t + 1):
            v += int(bits[tau]) << (KV * (t - tau))
        out.append(v % (1 << L))
    return out


@pytest.mark.parametrize("L,KV", [(16, 4), (12, 2), (9, 2), (7, 1), (10, 4)])
def test_walk_states_closed_form_and_c_decode(L, KV):
    rng = np.random.default_rng(L * 10 + KV)
    nc, nr, N = 3, 2, 37
    bits = rng.integers(0, 1 << KV, (nc, nr, N)).astype(np.uint8)
    start = rng.integers(0, 1 << L, (nc, nr)).astype(np.int32)
    w = O.walk_states(bits, start, L, KV)
    assert w.dtype == np.int64 and w.shape == (nc, nr, N)
    for j in range(nc):
        for i in range(nr):
            assert w[j, i].tolist() == _walk_closed_form(bits[j, i], start[j, i], L, KV)
    cb = rng.standard_normal((1 << L, 1)).astype(np.float32)
    walk_c, _ = O.decode(bits.reshape(nc * nr, N).astype(np.int32), start.reshape(-1), cb, L, KV)
    assert (walk_c.reshape(nc, nr, N) == w).all()


@pytest.mark.parametrize("m,n,V,Tx,Ty", [(32, 48, 2, 16, 16), (16, 16, 1, 16, 16), (24, 8, 2, 8, 4)])
def test_dequant_unit_matches_tiles_placed_by_slicing(m, n, V, Tx, Ty):
    L, KV = 10, 2 * V
    rng = np.random.default_rng(m + n + V)
    nc, nr, N = n // Ty, m // Tx, Tx * Ty // V
    bits = rng.integers(0, 1 << KV, (nc, nr, N)).astype(np.uint8)
    start = rng.integers(0, 1 << L, (nc, nr)).astype(np.int32)
    cb = rng.standard_normal((1 << L, V)).astype(np.float32)
    W = O.dequant_unit(bits, start, cb, (m, n), L, KV, Tx, Ty)
    walks = O.walk_states(bits, start, L, KV)
    ref = np.zeros((m, n))
    for j in range(nc):
        for i in range(nr):
            seq = cb[walks[j, i]].reshape(-1)  # step t, component v at t*V + v
            ref[i * Tx:(i + 1) * Tx, j * Ty:(j + 1) * Ty] = seq.reshape(Tx, Ty)
    assert W.dtype == np.float64
    assert (W == ref).all()


def test_dequant_target_scale_rounding_and_rht_round_trip():
    L, KV, V, Tx, Ty, m, n = 12, 4, 2, 16, 16, 64, 32
    rng = np.random.default_rng(3)
    nc, nr, N = n // Ty, m // Tx, Tx * Ty // V
    bits = rng.integers(0, 1 << KV, (nc, nr, N)).astype(np.uint8)
    start = rng.integers(0, 1 << L, (nc, nr)).astype(np.int32)
    cb = rng.standard_normal((1 << L, V)).astype(np.float32)
    sl = np.sign(rng.standard_normal(m)).astype(np.float32)
    sr = np.sign(rng.standard_normal(n)).astype(np.float32)
    W_scale = 0.0123456789012345
    unit = O.dequant_unit(bits, start, cb, (m, n), L, KV, Tx, Ty)
    tilde = (unit * W_scale).astype(np.float32)
    # one rounding of the exact product (then float64 -> float32) on a sample
    for x in unit.reshape(-1)[:200]:
        exact = Fraction(float(x)) * Fraction(W_scale)
        assert np.float32(float(np.float64(float(exact)))) == np.float32(float(np.float64(x) * W_scale))
    Wh = O.dequant_target(bits, start, cb, sl, sr, W_scale, (m, n), L, KV, Tx, Ty)
    assert Wh.shape == (m, n)
    assert (Wh == O.inverse_rht(tilde, sl, sr)).all()
    back = O.rht(Wh, sl, sr)
    np.testing.assert_allclose(back, tilde, rtol=0, atol=1e-6 * np.abs(tilde).max())


# ------------------------------ payload -----------------------------------

def _payload(rng, m=64, n=32, L=16, KV=4, V=2, Tx=16, Ty=16):
    nc, nr, N = n // Ty, m // Tx, Tx * Ty // V
    return dict(
        bitstreams=rng.integers(0, 1 << KV, (nc, nr, N)).astype(np.uint8),
        start_states=rng.integers(0, 1 << L, (nc, nr)).astype(np.int32),
        sign_l=np.sign(rng.standard_normal(m)).astype(np.float32),
        sign_r=np.sign(rng.standard_normal(n)).astype(np.float32),
        W_scale=0.0371, shape=(m, n),
        meta={"layer": 3, "kind": "attention", "proj": "q_proj"},
    )


def test_save_load_reference_payload(tmp_path):
    import bcjr
    p = _payload(np.random.default_rng(0))
    path = str(tmp_path / "L03" / "attn_q_proj.pt")
    bcjr.save_quantized(path, **p)
    d = bcjr.load_quantized(path)
    assert set(d) == {"bitstreams", "start_states", "sign_l", "sign_r", "W_scale", "shape", "meta", "config"}
    assert d["bitstreams"].dtype == np.uint8 and (d["bitstreams"] == p["bitstreams"]).all()
    assert d["start_states"].dtype == np.int32 and (d["start_states"] == p["start_states"]).all()
    assert d["sign_l"].dtype == np.int8 and (d["sign_l"] == p["sign_l"]).all()
    assert (d["sign_r"] == p["sign_r"]).all()
    assert d["W_scale"] == p["W_scale"] and d["shape"] == (64, 32)
    assert d["meta"] == p["meta"]
    assert d["config"] == {"L": 16, "k": 2, "V": 2, "Tx": 16, "Ty": 16}


class _Planted:
    """An object a payload must never be allowed to rebuild."""
    ran = False

    def __reduce__(self):
        return (_mark_ran, ())


def _mark_ran():
    _Planted.ran = True
    return 0


def test_load_refuses_payload_with_code(tmp_path):
    import bcjr
    path = str(tmp_path / "bad.pt")
    torch.save({"bitstreams": np.zeros((1, 1, 128), np.uint8), "extra": _Planted()}, path)
    with pytest.raises(pickle.UnpicklingError):
        bcjr.load_quantized(path)
    assert not _Planted.ran


def test_pack_layout_and_size():
    import bcjr
    rng = np.random.default_rng(1)
    for kV in (1, 2, 4):
        bits = rng.integers(0, 1 << kV, (3, 5, 128)).astype(np.uint8)
        packed = bcjr.pack_bitstreams(bits, kV)
        assert packed.shape == (3, 5, 128 * kV // 8)
        assert (packed.reshape(15, -1) == O.pack_bits(bits.reshape(15, 128), kV)).all()
        assert (bcjr.unpack_bitstreams(packed, 128, kV) == bits).all()
    # ragged: steps that do not fill the last byte
    bits = rng.integers(0, 4, (2, 7)).astype(np.uint8)
    packed = bcjr.pack_bitstreams(bits, 2)
    assert packed.shape == (2, 2)
    assert (packed == O.pack_bits(bits, 2)).all()
    assert (bcjr.unpack_bitstreams(packed, 7, 2) == bits).all()
    # hand-checked: steps 1, 2, 3, 0 at kV=2 -> 0b00_11_10_01
    assert bcjr.pack_bitstreams(np.array([[1, 2, 3, 0]], np.uint8), 2)[0, 0] == 0b00111001


def test_packed_file_round_trip(tmp_path):
    import bcjr
    from bcjr.serialize import bitstreams_of
    p = _payload(np.random.default_rng(2), m=256, n=128)
    path = str(tmp_path / "t.safetensors")
    bcjr.save_packed(path, **p)
    d = bcjr.load_quantized(path)  # dispatches on the extension
    assert d["packed"].shape == (128 // 16, 256 // 16, 64)
    assert (bitstreams_of(d) == p["bitstreams"]).all()
    assert d["W_scale"] == p["W_scale"] and d["shape"] == (256, 128) and d["meta"] == p["meta"]
    assert (d["sign_l"] == p["sign_l"]).all() and (d["start_states"] == p["start_states"]).all()
    # 2 bits per weight for the bitstream
    assert d["packed"].nbytes * 8 == 2 * 256 * 128
    assert os.path.getsize(path) < d["packed"].nbytes + 256 + 128 + 4 * 128 + 2048


def test_packed_loader_rejects_other_files(tmp_path):
    import bcjr
    from safetensors.numpy import save_file
    path = str(tmp_path / "w.safetensors")
    save_file({"weight": np.zeros((2, 2), np.float32)}, path)
    with pytest.raises(ValueError):
        bcjr.load_packed(path)


# ------------------------------ C ABI -------------------------------------

@pytest.fixture(scope="module")
def lib():
    import bcjr
    return bcjr.load_library()


@pytest.mark.parametrize("m,n,Tx,Ty,B,N,fmt,msg", [
    (32, 32, 16, 16, 4, 100, 0, "holds 256 weights"),
    (33, 32, 16, 16, 4, 128, 0, "whole number"),
    (32, 32, 16, 16, 3, 128, 0, "B=3"),
    (32, 32, 0, 16, 4, 128, 0, "tile 0x16"),
    (32, 32, 16, 16, 4, 128, 7, "format 7"),
    (32, 32, 16, 16, 4, 128, 2, "required"),
])
def test_dequant_validation_without_device(lib, m, n, Tx, Ty, B, N, fmt, msg):
    import bcjr._lib as BL
    p = BL.Problem(16, 2, 2, B, N, 0, 9, 0)
    rc = lib.bcjr_dequant(ctypes.byref(p), None, fmt, None, None, m, n, Tx, Ty, 1.0, None, None)
    assert rc == -1
    assert msg in lib.bcjr_last_error().decode()
