"""CPU tests of the C ABI library and the host-side logic (no GPU calls).

- libbcjr_hip.so loads and exports every function include/bcjr_hip.h declares;
- argument validation reports the right status without touching a device;
- the Python surface keeps the reference's assertion behaviour and layouts.
"""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "bcjr_hip.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(bcjr_\w+)\s*\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def lib():
    import bcjr
    path = bcjr.LIB_PATH
    if not os.path.exists(path):
        pytest.fail(f"{path} missing: run __graft_entry__.build()")
    return bcjr.load_library()


def test_header_and_binding_agree():
    import bcjr._lib as L
    assert _declared_functions() == sorted(L.EXPORTS)


def test_library_exports_every_declared_symbol(lib):
    for name in _declared_functions():
        assert hasattr(lib, name), name
    out = os.popen(f"nm -D --defined-only {lib._name}").read()
    for name in _declared_functions():
        assert re.search(rf"\bT {name}\b", out), name


def test_strerror_and_version(lib):
    assert lib.bcjr_version().startswith(b"bcjr_hip")
    assert lib.bcjr_strerror(0) == b"ok"
    assert lib.bcjr_strerror(-1) == b"invalid argument"
    assert lib.bcjr_strerror(-3) == b"workspace too small"
    assert lib.bcjr_strerror(12345) == b"unknown status"


@pytest.mark.parametrize("L,k,V,code,Q,B,N,status,msg", [
    (16, 3, 1, 0, 9, 4, 256, -2, "k*V=3"),
    (17, 2, 1, 0, 9, 4, 256, -2, "L=17"),
    (3, 2, 1, 0, 9, 4, 256, -2, "L=3"),
    (12, 1, 1, 0, 9, 4, 256, -2, "k*V=1 supports L <= 11"),
    (10, 1, 1, 2, 9, 4, 256, -2, "table code only"),
    (16, 2, 3, 0, 9, 4, 256, -1, "V=3"),
    (16, 2, 1, 0, 9, -1, 256, -1, "B=-1"),
    (16, 2, 1, 0, 9, 4, 0, -1, "N=0"),
    (16, 2, 1, 0, 9, 4, 5000, -1, "N=5000"),
    (16, 2, 2, 1, 9, 4, 128, -1, "1MAD/3INST codes are scalar"),
    (16, 2, 1, 3, 9, 4, 256, -1, "HYB code is 2-D"),
    (16, 2, 2, 3, 13, 4, 128, -1, "HYB Q=13"),
    (16, 2, 1, 7, 9, 4, 256, -1, "unknown code 7"),
])
def test_validation_without_device(lib, L, k, V, code, Q, B, N, status, msg):
    import bcjr._lib as BL
    p = BL.Problem(L, k, V, B, N, code, Q, 0)
    n = ctypes.c_size_t(0)
    rc = lib.bcjr_workspace_bytes(ctypes.byref(p), 0, ctypes.byref(n))
    assert rc == status
    assert msg in lib.bcjr_last_error().decode()


def test_null_problem(lib):
    n = ctypes.c_size_t(0)
    assert lib.bcjr_workspace_bytes(None, 0, ctypes.byref(n)) == -1
    assert lib.bcjr_forward(None, None, None, None, None, None, None, 0, None) == -1


# ------------------------------ host logic --------------------------------

def test_pred_succ_tables_closed_form():
    from bcjr import build_pred_succ_tables
    import oracle as O
    for L, k, V in [(16, 2, 2), (12, 2, 1), (6, 1, 1)]:
        p, s = build_pred_succ_tables(L, k, V, device="cpu")
        po, so = O.pred_succ_tables(L, k * V)
        assert (p.numpy() == po).all() and (s.numpy() == so).all()
        # every successor of s has s among its predecessors
        S = 1 << L
        idx = np.random.default_rng(0).integers(0, S, 64)
        for st in idx:
            for nxt in s[st].tolist():
                assert st in p[nxt].tolist()


def test_tile_untile_layout():
    """(m,n) -> sequences in block order col_block*n_row + row_block, 16x16 row-major
    (src/qat/ste.py:76-110 numpy form)."""
    from bcjr.quant import tile_for_viterbi, untile_from_viterbi
    m, n = 64, 48
    W = torch.arange(m * n, dtype=torch.float32).reshape(m, n)
    seqs, info = tile_for_viterbi(W)
    assert info == (m // 16, n // 16)
    Wn = W.numpy()
    for j in range(n // 16):
        for i in range(m // 16):
            tile = Wn[i * 16:(i + 1) * 16, j * 16:(j + 1) * 16].reshape(-1)
            assert (seqs[j * (m // 16) + i].numpy() == tile).all()
    assert torch.equal(untile_from_viterbi(seqs, info, (m, n)), W)


def test_python_surface_asserts_like_reference():
    from bcjr import bcjr_forward_backward
    seq = torch.zeros(2, 8, 2)
    cb = torch.zeros(1 << 6, 2)
    with pytest.raises(AssertionError):
        bcjr_forward_backward(torch.zeros(2, 8), cb, 1.0, L=6, k=2, V=2)
    with pytest.raises(AssertionError):
        bcjr_forward_backward(seq, torch.zeros(10, 2), 1.0, L=6, k=2, V=2)
    with pytest.raises(AssertionError):  # CPU tensors: the node runs only on the GPU
        bcjr_forward_backward(seq, cb, 1.0, L=6, k=2, V=2)


@pytest.mark.parametrize("m,n,msg", [
    (3, 64, "m=3"), (0, 64, "m=0"), (32768, 64, "m=32768"),
    (64, 0, "n=0"), (64, 96, "n=96"), (64, 32768, "n=32768"),
])
def test_rht_validation_without_device(lib, m, n, msg):
    dummy = ctypes.c_void_p(16)  # never dereferenced: the shape check fails first
    assert lib.bcjr_rht(dummy, ctypes.c_void_p(32), m, n, dummy, dummy, 0, None) == -1
    assert msg in lib.bcjr_last_error().decode()


def test_rht_rejects_null_and_alias(lib):
    p = ctypes.c_void_p(16)
    assert lib.bcjr_rht(None, p, 64, 64, p, p, 0, None) == -1
    assert "non-NULL" in lib.bcjr_last_error().decode()
    assert lib.bcjr_rht(p, p, 64, 64, ctypes.c_void_p(32), ctypes.c_void_p(48), 1, None) == -1
    assert "alias" in lib.bcjr_last_error().decode()


def test_hadamard_validation_without_device(lib):
    assert lib.bcjr_hadamard(None, None, 4, 48, 1.0, None) == -1
    assert "n=48" in lib.bcjr_last_error().decode()
    assert lib.bcjr_hadamard(None, None, -1, 64, 1.0, None) == -1
    assert lib.bcjr_hadamard(None, None, 0, 64, 1.0, None) == 0   # nothing to do
    assert lib.bcjr_hadamard(None, None, 2, 64, 1.0, None) == -1
    assert "non-NULL" in lib.bcjr_last_error().decode()


def test_sign_vector_generator_matches_reference_draw():
    # src/rht/transform.py:58-62: default_rng(seed).choice([-1.0, 1.0], size=n) as float32
    import bcjr
    s = bcjr.make_sign_vector(1000, 7)
    ref = np.random.default_rng(7).choice([-1.0, 1.0], size=1000).astype(np.float32)
    assert s.dtype == np.float32 and np.array_equal(s, ref)


def test_rht_batched_validation_without_device(lib):
    p = ctypes.c_void_p(16)
    assert lib.bcjr_rht_batched(p, ctypes.c_void_p(1 << 20), -1, 64, 64, p, p, 0, None) == -1
    assert "batch=-1" in lib.bcjr_last_error().decode()
    assert lib.bcjr_rht_batched(None, None, 0, 64, 64, None, None, 0, None) == 0  # nothing to do
    assert lib.bcjr_rht_batched(p, p, 2, 64, 48, p, p, 0, None) == -1
    assert "n=48" in lib.bcjr_last_error().decode()
    # out overlapping the second matrix of W
    assert lib.bcjr_rht_batched(ctypes.c_void_p(4096), ctypes.c_void_p(4096 + 64 * 64 * 4), 2, 64, 64, p, p, 0,
                                None) == -1
    assert "alias" in lib.bcjr_last_error().decode()


def test_expert_dispatch_validates_before_device():
    import bcjr
    W = [torch.zeros(64, 64), torch.zeros(64, 40)]
    s = [torch.ones(64), torch.ones(64)]
    with pytest.raises(AssertionError, match="not tileable"):
        bcjr.bcjr_quantize_experts(W, s, [torch.ones(64), torch.ones(40)], None, 0.1)
    with pytest.raises(AssertionError, match="sign vectors"):
        bcjr.bcjr_quantize_experts(W, s[:1], s, None, 0.1)
    with pytest.raises(AssertionError, match="expected 1 or 2"):
        bcjr.bcjr_quantize_experts([torch.zeros(64, 64)] * 2, s, s, None, [0.1, 0.2, 0.3])
    assert bcjr.bcjr_quantize_experts([], [], [], None, 0.1) == []


def test_cosine_temperature_schedule():
    """anneal.py:53-61: T_0 at step 0, T_min from the last step on."""
    from bcjr import cosine_temperature_schedule as sched
    assert sched(0, 100, 1.0, 0.01) == 1.0
    assert abs(sched(99, 100, 1.0, 0.01) - 0.01) < 1e-15
    assert sched(500, 100, 1.0, 0.01) == sched(99, 100, 1.0, 0.01)
    assert sched(-3, 100, 1.0, 0.01) == 1.0
    assert sched(5, 1, 1.0, 0.01) == 0.01
    mid = sched(50, 101, 2.0, 0.0)  # cos(pi/2) = 0: the midpoint is the mean
    assert abs(mid - 1.0) < 1e-12


def test_precompute_tables_match_reference_loops():
    """precompute_predecessors(_v) and precompute_codebook_v against the loops of
    src/viterbi/encode.py:22-37, 218-247 restated on a small trellis."""
    from bcjr import encode as E
    for L, k, V in [(6, 2, 1), (8, 1, 2), (8, 2, 2)]:
        kV = k * V
        ref = np.zeros((1 << L, 1 << kV), np.int32)
        for s in range(1 << L):
            for p in range(1 << kV):
                ref[s, p] = (p << (L - kV)) | (s >> kV)
        got = E.precompute_predecessors_v(L, k, V)
        assert got.dtype == np.int32 and np.array_equal(got, ref)
    assert np.array_equal(E.precompute_predecessors(6, 2), E.precompute_predecessors_v(6, 2, 1))
    cb = E.precompute_codebook_v(4, 2, lambda s: np.stack([s * 0.5, -(s * 1.0)], 1))
    assert cb.dtype == np.float32 and cb.shape == (16, 2) and cb[3, 1] == -3.0
    with pytest.raises(AssertionError, match="expected"):
        E.precompute_codebook_v(4, 2, lambda s: s * 1.0)



@pytest.mark.parametrize("Q", [3, 6, 9])
def test_hyb_column_walk_identity(Q):
    """The soft kernels' HYB column walk at L=16, kV=4: for every state
    s = p*4096 + r, the float2 at byte col_base(r) + ((p*(2r+1)) mod 16) * 512 of
    the 32 x 64 staged table is signed LUT entry bits [15-Q, 16) of s^2 + s
    (src/qat/ste.py:376-392), without passing row 31."""
    s = np.arange(1 << 16, dtype=np.uint64)
    x = (s * s + s) & 0xFFFFFFFF
    idx = (x >> (15 - Q)) & ((2 << Q) - 1)
    p, r = s >> 12, s & 4095
    x0 = (r * r + r) & 0xFFFFFFFF
    base = (((x0 >> (15 - Q)) & ((1 << (Q - 3)) - 1)) << 3) | (((x0 >> 12) & 15) << 9)
    byte = base + (((p * (2 * (r & 7) + 1)) & 15) << 9)
    row, col = byte >> 9, (byte >> 3) & 63
    assert row.max() < 32 and (byte & 7).max() == 0
    assert np.array_equal(col + (1 << (Q - 3)) * (row & 15), idx)



def _col_walk_maps():
    """The lane and layout maps of the column-walk kernels, evaluated from their
    one-line definitions in bcjr_device.h and the swizzle constant in
    bcjr_capi.hip (so the checks below follow the source)."""
    csrc = os.path.join(ROOT, "quant-2bit_amd", "csrc")
    dev = open(os.path.join(csrc, "bcjr_device.h")).read()
    maps = {}
    for name in ("col_walk_unit", "col_walk_state_el"):
        m = re.search(name + r"\(uint32_t (\w+)\) \{\s*return ([^;]+);", dev)
        assert m, name
        body = re.sub(r"(\d+)u\b", r"\1", m.group(2))
        maps[name] = eval(f"lambda {m.group(1)}: {body}")
    capi = open(os.path.join(csrc, "bcjr_capi.hip")).read()
    m = re.search(r"kColWalkSwizzle = \{\{([^}]*)\}, \{([^}]*)\}\}", capi)
    assert m
    shifts = [int(a) for a in m.group(1).split(",")]
    masks = [int(a.strip().rstrip("u")) for a in m.group(2).split(",")]
    maps["swizzle"] = lambda x: x ^ np.bitwise_xor.reduce([(x >> a) & k for a, k in zip(shifts, masks)])
    return maps


def _distinct_in_groups(el, group, banks):
    el = np.asarray(el).reshape(-1, group) % banks
    return all(len(set(g.tolist())) == group for g in el)


def test_column_walk_layouts_are_bank_conflict_free():
    """Column-walk soft kernels (L=16, kV=4, 256 threads, thread tid on butterfly
    u = col_walk_unit(tid)), under gfx950's LDS banking: 64-bit reads serve each
    half-wave from 32 eight-byte banks, 64-bit writes each quarter-wave from 32
    four-byte banks, 32-bit reads 64 lanes from 64 banks, 32-bit writes 32 lanes
    from 32 banks.  Checked: the LUT gathers at Q = 9 (bank = bits [6, 11) of
    r^2 + r, r = 16u + c), the 32-bit reads of the per-step emission tables in
    the LUT's layout (bank = bits [6, 12)), and the in-place state vectors at the
    rotations 0, 4, 8: the forward's floats (col_walk_state_el, 32-bit) and the
    backward's swizzled (m~, mu) pairs (64-bit)."""
    M = _col_walk_maps()
    tid = np.arange(256, dtype=np.int64)
    U = M["col_walk_unit"](tid)
    assert sorted(U.tolist()) == list(range(256))
    lut_bank = lambda r: ((r * r + r) >> 6) & 31
    table_bank = lambda r: ((r * r + r) >> 6) & 63
    for c in range(16):
        assert _distinct_in_groups(lut_bank(16 * U + c), 32, 32), c
        assert _distinct_in_groups(table_bank(16 * U + c), 64, 64), c
    # the lane map is what makes the gathers conflict-free: u = tid collides
    assert not _distinct_in_groups(lut_bank(16 * tid), 32, 32)

    j = np.arange(4096, dtype=np.int64)
    rotr = lambda x, rho: ((x | (x << 12)) >> rho) & 4095
    # in place: butterfly u's outputs 16u + r of one step are its inputs r*256 + u
    # of the next, one rotation by kV = 4 later
    for r in range(16):
        assert np.array_equal(rotr(16 * U + r, 4), 256 * r + U)
    E, S = M["col_walk_state_el"], M["swizzle"]
    for layout in (E, S):
        assert sorted(layout(j).tolist()) == list(range(4096))
    for rho in (0, 4, 8):
        for k in range(16):
            x = rotr(256 * k + U, rho)
            # the split the forward addresses with: element of u XOR element of k*256
            assert np.array_equal(E(x), E(rotr(U, rho)) ^ E(rotr(np.full_like(U, 256 * k), rho)))
            assert _distinct_in_groups(E(x), 64, 64) and _distinct_in_groups(E(x), 32, 32), (rho, k)
            assert _distinct_in_groups(S(x), 32, 32) and _distinct_in_groups(S(x), 16, 16), (rho, k)


# ------------------------- contract checks (no device) -------------------------

@pytest.mark.parametrize("op", ["forward", "backward", "viterbi", "viterbi_constrained", "forward_entropy"])
def test_undersized_workspace_is_reported_before_any_device_call(lib, op):
    """BCJR_EWORKSPACE through a real call: the slot size depends on the problem
    alone, so the status comes back on a machine without a GPU.  The pointers
    are never dereferenced."""
    import bcjr._lib as BL
    p = BL.Problem(16, 2, 1, 4, 256, 2, 9, 0)
    d = ctypes.c_void_p(4096)
    ws_small = 100
    if op == "forward":
        rc = lib.bcjr_forward(ctypes.byref(p), d, d, None, d, None, d, ws_small, None)
        slot = 256 * (1 << 14) * 4
    elif op == "forward_entropy":
        rc = lib.bcjr_forward_entropy(ctypes.byref(p), d, d, None, d, None, d, d, ws_small, None)
        slot = 256 * (1 << 14) * 4
    elif op == "backward":
        rc = lib.bcjr_backward(ctypes.byref(p), d, d, None, None, d, None, d, d, ws_small, None)
        slot = 256 * (1 << 14) * 8
    elif op == "viterbi":
        rc = lib.bcjr_viterbi(ctypes.byref(p), d, None, None, None, None, None, None, None, d, ws_small, None)
        slot = 256 * (1 << 14)
    else:
        rc = lib.bcjr_viterbi_constrained(ctypes.byref(p), d, None, 4, d, None, None, None, None, None, None,
                                          d, ws_small, None)
        slot = 256 * (1 << 14)
    assert rc == BL.BCJR_EWORKSPACE
    msg = lib.bcjr_last_error().decode()
    assert f"({slot} bytes)" in msg and "100 bytes" in msg


@pytest.mark.parametrize("op", ["forward", "forward_entropy", "backward", "viterbi", "viterbi_constrained"])
def test_missing_pointers_are_reported_before_any_device_call(lib, op):
    """A null input or output, a table code without its table, an unsupported
    k*V or an overlap wider than L - k*V: refused on the host, before the launch
    plan queries the device."""
    import bcjr._lib as BL
    d = ctypes.c_void_p(4096)
    big = 1 << 40
    p = BL.Problem(16, 2, 1, 4, 256, 0, 9, 0)  # table code
    if op == "forward":
        calls = [(lambda: lib.bcjr_forward(ctypes.byref(p), None, d, d, d, None, d, big, None), "non-NULL"),
                 (lambda: lib.bcjr_forward(ctypes.byref(p), d, d, None, d, None, d, big, None), "codebook")]
    elif op == "forward_entropy":
        calls = [(lambda: lib.bcjr_forward_entropy(ctypes.byref(p), d, d, d, d, None, None, d, big, None),
                  "non-NULL")]
    elif op == "backward":
        calls = [(lambda: lib.bcjr_backward(ctypes.byref(p), d, d, d, None, None, None, d, d, big, None),
                  "non-NULL"),
                 (lambda: lib.bcjr_backward(ctypes.byref(p), d, d, None, None, d, None, d, d, big, None),
                  "codebook")]
    elif op == "viterbi":
        p3 = BL.Problem(12, 3, 1, 4, 64, 0, 9, 0)
        calls = [(lambda: lib.bcjr_viterbi(ctypes.byref(p), None, d, None, None, None, None, None, None, d, big,
                                           None), "non-NULL"),
                 (lambda: lib.bcjr_viterbi(ctypes.byref(p), d, None, None, None, None, None, None, None, d, big,
                                           None), "codebook"),
                 (lambda: lib.bcjr_viterbi(ctypes.byref(p3), d, d, None, None, None, None, None, d, d, big, None),
                  "k*V=3")]
    else:
        calls = [(lambda: lib.bcjr_viterbi_constrained(ctypes.byref(p), d, d, 15, d, None, None, None, None, None,
                                                       None, d, big, None), "overlap_bits=15"),
                 (lambda: lib.bcjr_viterbi_constrained(ctypes.byref(p), d, d, 4, None, None, None, None, None,
                                                       None, None, d, big, None), "non-NULL")]
    for call, msg in calls:
        rc = call()
        assert rc in (BL.BCJR_EINVAL, BL.BCJR_EUNSUPPORTED), (rc, lib.bcjr_last_error())
        assert msg in lib.bcjr_last_error().decode()


def test_viterbi_trace_validates_before_any_device_call(lib):
    """bcjr_viterbi_trace refuses bad problems and missing pointers on the host
    (no device needed), and an empty batch is a no-op."""
    import bcjr._lib as BL
    d = ctypes.c_void_p(4096)
    p = BL.Problem(16, 2, 1, 2, 64, 0, 9, 0)
    assert lib.bcjr_viterbi_trace(ctypes.byref(p), d, d, None, d, None) == BL.BCJR_EINVAL
    assert "non-NULL" in lib.bcjr_last_error().decode()
    assert lib.bcjr_viterbi_trace(ctypes.byref(p), d, None, d, d, None) == BL.BCJR_EINVAL
    assert "codebook" in lib.bcjr_last_error().decode()
    p = BL.Problem(17, 2, 1, 2, 64, 0, 9, 0)
    assert lib.bcjr_viterbi_trace(ctypes.byref(p), d, d, d, d, None) == BL.BCJR_EUNSUPPORTED
    p = BL.Problem(16, 2, 1, 0, 64, 2, 9, 0)
    assert lib.bcjr_viterbi_trace(ctypes.byref(p), None, None, None, None, None) == BL.BCJR_OK


def test_workspace_check_passes_for_empty_batch(lib):
    import bcjr._lib as BL
    p = BL.Problem(16, 2, 1, 0, 256, 2, 9, 0)
    assert lib.bcjr_forward(ctypes.byref(p), None, None, None, None, None, None, 0, None) == 0


def test_codebook_device_mismatch_is_an_assertion():
    """A codebook (or LUT, bitstream, start state) on another device than the
    launch raises AssertionError before any pointer reaches a kernel."""
    from bcjr.codes import resolve_codebook
    from bcjr import ops
    cb = torch.zeros(1 << 12, 1)
    with pytest.raises(AssertionError, match="codebook is on cpu"):
        resolve_codebook(cb, 12, 2, 1, torch.device("cuda:0"))
    with pytest.raises(AssertionError, match="codebook"):
        resolve_codebook(torch.zeros(10, 1), 12, 2, 1, torch.device("cuda:0"))
    with pytest.raises(AssertionError, match="bitstream is on cpu"):
        ops._on(torch.device("cuda:0"), codebook_or_lut=None, bitstream=torch.zeros(4, dtype=torch.int32))
    meta = torch.empty(4, device="meta")
    with pytest.raises(AssertionError, match="packed is on meta"):
        ops._on(torch.device("cpu"), packed=meta)
    ops._on(torch.device("cpu"), packed=torch.zeros(2), codebook_or_lut=None)


def test_tagged_hyb_lut_device_is_checked():
    from bcjr.codes import _tag, resolve_codebook
    cb = _tag(torch.zeros(1 << 8, 2, device="meta"), 3, torch.zeros(1 << 9, 2), 9)
    with pytest.raises(AssertionError, match="HYB LUT is on cpu"):
        resolve_codebook(cb, 8, 1, 2, torch.device("meta"))


def test_one_bit_per_step_takes_the_table_kernels():
    """k*V = 1 has table kernels only: a codebook tagged (or recognisable) as a
    generator's output is handed to them as a table, not as a generator code
    the library would refuse."""
    from bcjr.codes import _tag, resolve_codebook
    from bcjr._lib import CODE_3INST, CODE_TABLE
    cb = _tag(torch.randn(1 << 6, 1), CODE_3INST)
    spec, table = resolve_codebook(cb, 6, 1, 1, torch.device("cpu"))
    assert spec.code == CODE_TABLE and table.data_ptr() == cb.data_ptr()
    spec, table = resolve_codebook(cb, 6, 2, 1, torch.device("cpu"))
    assert spec.code == CODE_3INST and table is None


def test_registered_ops_have_fake_implementations():
    """The engine's torch operators are registered in C++ (libbcjr_torch.so,
    TORCH_LIBRARY) with Meta kernels, and the node (bcjr::node, bcjr::node_backward)
    in Python over them: fake tensors give every output shape without a device."""
    from torch._subclasses.fake_tensor import FakeTensorMode
    import bcjr  # noqa: F401  (loads the operator library, registers the node)
    from bcjr import _lib
    assert _lib._ops_loaded and os.path.exists(_lib.OPS_PATH)
    for name in ("forward", "forward_internals", "forward_entropy", "backward", "viterbi", "decode", "viterbi_trace",
                 "dequant", "codebook", "hadamard", "rht", "rht_batched"):
        assert torch._C._dispatch_has_kernel_for_dispatch_key(f"bcjr::{name}", "CUDA"), name
        assert torch._C._dispatch_has_kernel_for_dispatch_key(f"bcjr::{name}", "Meta"), name
    with FakeTensorMode():
        seq = torch.empty(5, 32, 1)
        cb = torch.empty(1 << 8, 1)
        T = torch.empty(1)
        soft, logZ = torch.ops.bcjr.node(seq, cb, T, 8, 2, 1)
        assert soft.shape == (5, 32, 1) and logZ.shape == (5,) and soft.dtype == torch.float32
        d = torch.ops.bcjr.node_backward(seq, cb, T, torch.empty(5, 32, 1), None, 8, 2, 1)
        assert d.shape == (5, 32, 1)
        soft, logZ = torch.ops.bcjr.forward(seq, T, None, 8, 2, 1, _lib.CODE_3INST, 9)
        assert soft.shape == (5, 32, 1) and logZ.shape == (5,)
        assert torch.ops.bcjr.backward(seq, T, None, seq, None, 8, 2, 1, _lib.CODE_3INST, 9).shape == (5, 32, 1)
        outs = torch.ops.bcjr.forward_internals(seq, T, cb, 8, 2, 1, _lib.CODE_TABLE, 9)
        assert [tuple(o.shape) for o in outs] == [(5, 32, 1), (5,), (5, 32, 256), (5, 32, 256), (5, 32, 256)]
        walk, bits, start, recon, mse, packed = torch.ops.bcjr.viterbi(seq, None, 8, 2, 1, _lib.CODE_3INST, 9, True)
        assert walk.shape == bits.shape == (5, 32) and start.shape == (5,) and recon.shape == (5, 32, 1)
        assert packed.shape == (5, 8) and packed.dtype == torch.uint8 and walk.dtype == torch.int32
        assert torch.ops.bcjr.dequant(torch.empty(4, dtype=torch.int32), None, None, torch.empty(4, 64, dtype=torch.uint8),
                                      32, 32, 16, 16, 1.0, 8, 2, 1, _lib.CODE_3INST, 9).shape == (32, 32)
        assert torch.ops.bcjr.codebook(torch.empty(0), None, 8, _lib.CODE_1MAD, 9).shape == (256, 1)
        W = torch.empty(64, 32)
        out = torch.ops.bcjr.rht(W, torch.empty(64), torch.empty(32), False)
        assert out.shape == (64, 32)
        h = torch.ops.bcjr.hadamard(torch.empty(3, 16), 0.25)
        assert h.shape == (3, 16)


def test_temperature_tensor_has_no_host_copy_for_python_floats():
    from bcjr.forward_backward import temperature_tensor
    t = temperature_tensor(0.25, torch.device("cpu"))
    assert t.shape == (1,) and t.dtype == torch.float32 and float(t) == 0.25
    tb = temperature_tensor(torch.tensor([0.1, 0.2], dtype=torch.float64), torch.device("cpu"))
    assert tb.dtype == torch.float32 and tb.shape == (2,)
