"""bcjr_forward_noalloc (the entry point that allocates nothing) against
bcjr_forward through the C ABI: two calls in a row, the second with a smaller
input, each bit-identical to the allocating entry point's output (the same
kernel runs every sequence independently; only the number of slots differs).
Also: a problem whose slot exceeds the static array is refused, and the array
is reserved on a GPU only by the first no-alloc call there, not by loading the
library or by the other entry points."""
import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[no-alloc] {msg}", flush=True)


def _call(lib, prob, seq, T, table, soft, logZ, ws=None):
    from bcjr import _lib
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if ws is None:
        rc = lib.bcjr_forward_noalloc(ctypes.byref(prob), seq.data_ptr(), T.data_ptr(), _lib.ptr(table),
                                      soft.data_ptr(), logZ.data_ptr(), stream)
    else:
        rc = lib.bcjr_forward(ctypes.byref(prob), seq.data_ptr(), T.data_ptr(), _lib.ptr(table), soft.data_ptr(),
                              logZ.data_ptr(), ws.data_ptr(), ws.numel(), stream)
    _lib.check(rc, "forward")


@pytest.mark.parametrize("L,k,V,N,Bs,code", [(16, 2, 1, 256, (37, 5), "3inst"), (12, 2, 1, 256, (300, 17), "1mad"),
                                             (12, 2, 2, 128, (20, 3), "hyb")])
def test_noalloc_matches_forward(bcjr_mod, L, k, V, N, Bs, code):
    from bcjr import _lib
    from bcjr.codes import resolve_codebook
    lib = _lib.load()
    dev = torch.device("cuda")
    if code == "3inst":
        cb = bcjr_mod.make_3inst_codebook(L, dev)
    elif code == "1mad":
        cb = bcjr_mod.make_1mad_codebook(L, dev)
    else:
        lut = np.random.default_rng(1).standard_normal((512, 2)).astype(np.float32)
        cb = bcjr_mod.make_hyb_codebook_gpu(lut, 9, L, dev)
    spec, table = resolve_codebook(cb, L, k, V, dev)
    for call, B in enumerate(Bs):
        _say(f"L={L} {code} N={N} call {call} B={B}")
        x = torch.randn(B, N, V, device=dev, generator=torch.Generator(dev).manual_seed(B))
        T = torch.rand(B, device=dev, generator=torch.Generator(dev).manual_seed(B + 1)) * 0.5 + 0.05
        prob = spec.problem(B, N, True)
        nbytes = ctypes.c_size_t(0)
        _lib.check(lib.bcjr_workspace_bytes(ctypes.byref(prob), 0, ctypes.byref(nbytes)), "ws")
        ws = torch.empty(nbytes.value, dtype=torch.uint8, device=dev)
        soft_a = torch.full((B, N, V), 7.0, device=dev)
        logZ_a = torch.full((B,), 7.0, device=dev)
        soft_b = torch.full((B, N, V), -7.0, device=dev)
        logZ_b = torch.full((B,), -7.0, device=dev)
        _call(lib, prob, x, T, table, soft_a, logZ_a, ws=ws)
        _call(lib, prob, x, T, table, soft_b, logZ_b)
        torch.cuda.synchronize()
        assert torch.equal(soft_a, soft_b) and torch.equal(logZ_a, logZ_b)
        assert torch.isfinite(soft_b).all()


def test_noalloc_refuses_a_slot_larger_than_the_array(bcjr_mod):
    from bcjr import _lib
    lib = _lib.load()
    prob = _lib.Problem(16, 2, 1, 1, 2049, _lib.CODE_3INST, 9, 0)  # 2049 * 16384 * 4 B > 128 MiB
    d = torch.zeros(2049, device="cuda")
    rc = lib.bcjr_forward_noalloc(ctypes.byref(prob), d.data_ptr(), d.data_ptr(), None, d.data_ptr(),
                                  d.data_ptr(), None)
    assert rc == _lib.BCJR_EWORKSPACE
    assert "static scratch holds 134217728" in lib.bcjr_last_error().decode()


# Run in a fresh process, so that no earlier test has called the no-alloc entry
# point: device memory free before and after a bcjr_forward, then after the
# first and a second bcjr_forward_noalloc, with every tensor allocated first.
_RESERVE_PROBE = r"""
import ctypes, sys
sys.path.insert(0, sys.argv[1])
import torch
from bcjr import _lib
dev = torch.device("cuda")
def free():
    torch.cuda.synchronize()
    return torch.cuda.mem_get_info(dev)[0]
lib = _lib.load()
L, N, B = 12, 64, 4
prob = _lib.Problem(L, 2, 1, B, N, _lib.CODE_1MAD, 9, 0)
x = torch.randn(B, N, 1, device=dev)
T = torch.full((1,), 0.2, device=dev)
soft, logZ = torch.empty_like(x), torch.empty(B, device=dev)
n = ctypes.c_size_t(0)
_lib.check(lib.bcjr_workspace_bytes(ctypes.byref(prob), 0, ctypes.byref(n)), "ws")
ws = torch.empty(n.value, dtype=torch.uint8, device=dev)
s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
f0 = free()
_lib.check(lib.bcjr_forward(ctypes.byref(prob), x.data_ptr(), T.data_ptr(), None, soft.data_ptr(),
                            logZ.data_ptr(), ws.data_ptr(), ws.numel(), s), "forward")
f1 = free()
def noalloc():
    _lib.check(lib.bcjr_forward_noalloc(ctypes.byref(prob), x.data_ptr(), T.data_ptr(), None,
                                        soft.data_ptr(), logZ.data_ptr(), s), "forward_noalloc")
noalloc()
f2 = free()
noalloc()
f3 = free()
print("RESERVED", f0 - f1, f1 - f2, f2 - f3, flush=True)
"""


def test_noalloc_array_reserved_by_its_first_call():
    if os.environ.get("HIP_ENABLE_DEFERRED_LOADING", "1") == "0":
        pytest.skip("code objects load eagerly in this environment")
    pkg = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "quant-2bit_amd")
    _say("fresh process: free device memory around forward and two no-alloc calls")
    out = subprocess.run([sys.executable, "-c", _RESERVE_PROBE, pkg], capture_output=True, text=True,
                         timeout=240)
    assert out.returncode == 0, out.stderr[-2000:]
    line = [ln for ln in out.stdout.splitlines() if ln.startswith("RESERVED")][-1]
    fwd, first, second = (int(v) for v in line.split()[1:])
    _say(f"forward {fwd >> 20} MiB, first no-alloc call {first >> 20} MiB, second {second >> 20} MiB")
    scratch = 128 << 20
    assert fwd < scratch // 4  # the allocating forward does not load the array
    assert first >= scratch  # the first no-alloc call does
    assert second < scratch // 4  # and later calls reuse it
