"""GPU tests of the node's contract beyond parity:

  * codebooks made outside bcjr.codes (the reference's own HYB construction, a
    .clone(), a .to() copy) reach the hashed / LUT kernels, and a perturbed
    table reaches the table kernels, with results identical to the tagged path;
  * non-finite or non-positive T, and non-finite weights or upstream gradients,
    give NaN outputs for exactly the affected sequences;
  * return_internals=True keeps soft and log Z differentiable;
  * a python-float T is capture-safe (fill kernel, no host copy): a captured
    forward + backward replays to the eager result;
  * torch.compile(fullgraph=True) traces bcjr_quantize_weight (RHT, tiles,
    node, inverse RHT) without a graph break, matching eager (the reference's
    compile gate, src/tripwires/test_bcjr_compile.py:28-84).
"""
import numpy as np
import pytest
import torch

from conftest import max_rel

pytestmark = pytest.mark.gpu

SOFT_TOL, GRAD_TOL = 1e-4, 1e-3


def _say(msg):
    print(f"[gpu-contract] {msg}", flush=True)


def _reference_style_hyb_table(lut, Q, L, dev):
    """The (2^L, 2) HYB table built with plain torch ops the way the reference's
    make_hyb_codebook_gpu defines it (src/qat/ste.py:376-392): no generator tag."""
    s = torch.arange(1 << L, dtype=torch.int64, device=dev)
    x = (s * s + s) & 0xFFFFFFFF
    idx = (x >> (15 - Q)) & ((1 << Q) - 1)
    neg = ((x >> 15) & 1).bool()
    cb = lut[idx].clone()
    cb[:, 1] = torch.where(neg, -cb[:, 1], cb[:, 1])
    return cb.contiguous()


@pytest.mark.parametrize("L,k,V,N,kind", [(16, 2, 2, 128, "hyb"), (12, 2, 2, 64, "hyb"), (12, 2, 1, 64, "3inst"),
                                          (12, 2, 1, 64, "1mad")])
def test_untagged_codebooks_reach_the_generator_kernels(bcjr_mod, L, k, V, N, kind):
    _say(f"recognition L={L} {kind}")
    from bcjr import ops
    from bcjr.codes import resolve_codebook
    dev = torch.device("cuda")
    if kind == "hyb":
        lut = torch.tensor(np.random.default_rng(5).standard_normal((512, 2)).astype(np.float32), device=dev)
        tagged = bcjr_mod.make_hyb_codebook_gpu(lut, 9, L, dev)
        plain = _reference_style_hyb_table(lut, 9, L, dev)
        assert torch.equal(plain, tagged)
        want = ops.CODE_HYB
    else:
        tagged = (bcjr_mod.make_3inst_codebook if kind == "3inst" else bcjr_mod.make_1mad_codebook)(L, dev)
        plain = tagged.clone()
        want = ops.CODE_3INST if kind == "3inst" else ops.CODE_1MAD
    assert not hasattr(plain, "_bcjr_code")
    spec, table = resolve_codebook(plain, L, k, V, dev)
    assert spec.code == want
    spec2, _ = resolve_codebook(plain[:, :].view(plain.shape), L, k, V, dev)  # a view shares the entry
    assert spec2.code == want
    x = torch.randn(6, N, V, device=dev, generator=torch.Generator(dev).manual_seed(1), requires_grad=True)
    g = torch.randn(6, N, V, device=dev, generator=torch.Generator(dev).manual_seed(2))
    outs = []
    for cb in (tagged, plain):
        xs = x.detach().clone().requires_grad_(True)
        soft, logZ = bcjr_mod.bcjr_forward_backward(xs, cb, 0.2, L=L, k=k, V=V)
        soft.backward(g)
        outs.append((soft.detach(), logZ.detach(), xs.grad))
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    # One entry changed: the table kernels run, unless the changed table is
    # itself exactly a HYB codebook of some LUT (a small L with a large Q can
    # represent almost any table), which then must regenerate it bit for bit.
    def _represents(cb):
        sp, tab = resolve_codebook(cb, L, k, V, dev)
        if sp.code == ops.CODE_TABLE:
            return tab.data_ptr() == cb.data_ptr()
        if sp.code == ops.CODE_HYB:
            return torch.equal(ops.codebook(ops.CODE_HYB, L, dev, lut=tab, Q=sp.Q), cb)
        return torch.equal(ops.codebook(sp.code, L, dev), cb)

    bad = plain.clone()
    bad[7, 0] += 0.5
    assert _represents(bad)
    if L == 16:
        assert resolve_codebook(bad, L, k, V, dev)[0].code == ops.CODE_TABLE
    # an in-place change of a recognised table is seen (its version moves)
    plain[3, 0] += 0.25
    assert _represents(plain)
    if L == 16 or kind != "hyb":
        assert resolve_codebook(plain, L, k, V, dev)[0].code == ops.CODE_TABLE


@pytest.mark.parametrize("L", [12, 14, 16])  # 512-thread forward; 1024-thread forward at 1 and 4 butterflies per thread
def test_non_finite_inputs_give_nan_for_their_sequences(bcjr_mod, oracle, L):
    _say(f"non-finite inputs L={L}")
    N, B = 64, 8
    cb = bcjr_mod.make_1mad_codebook(L, "cuda")
    cb_np = cb.cpu().numpy()
    rng = np.random.default_rng(3)
    seq = rng.standard_normal((B, N, 1)).astype(np.float32)
    g = rng.standard_normal((B, N, 1)).astype(np.float32)
    T = np.full(B, 0.2, dtype=np.float32)
    seq[1, 5, 0] = np.nan
    seq[2, 9, 0] = np.inf
    T[3], T[4], T[5] = 0.0, -0.5, np.inf
    g[6, 2, 0] = np.nan
    bad_fwd = {1, 2, 3, 4, 5}
    bad_bwd = bad_fwd | {6}
    x = torch.tensor(seq, device="cuda", requires_grad=True)
    soft, logZ = bcjr_mod.bcjr_forward_backward(x, cb, torch.tensor(T, device="cuda"), L=L, k=2, V=1)
    soft.backward(torch.tensor(g, device="cuda"))
    s, z, d = soft.detach().cpu().numpy(), logZ.detach().cpu().numpy(), x.grad.cpu().numpy()
    for b in range(B):
        if b in bad_fwd:
            assert np.isnan(s[b]).all() and np.isnan(z[b]), b
        else:
            s_ref, _ = oracle.bcjr_forward(seq[b:b + 1], cb_np, float(T[b]), L, 2)
            assert max_rel(s[b:b + 1], s_ref) < SOFT_TOL, b
        if b in bad_bwd:
            assert np.isnan(d[b]).all(), b
        else:
            d_ref = oracle.bcjr_backward(seq[b:b + 1], cb_np, float(T[b]), L, 2, g[b:b + 1])
            assert max_rel(d[b:b + 1], d_ref) < GRAD_TOL, b
    # a non-finite g_logZ poisons only its own sequence
    xs = torch.tensor(seq[[0, 7]], device="cuda", requires_grad=True)
    _, lz = bcjr_mod.bcjr_forward_backward(xs, cb, 0.2, L=L, k=2, V=1)
    lz.backward(torch.tensor([1.0, float("nan")], device="cuda"))
    gr = xs.grad.cpu().numpy()
    assert np.isfinite(gr[0]).all() and np.isnan(gr[1]).all()
    # the same rules on a python-float T
    soft0, logZ0 = bcjr_mod.bcjr_forward_backward(torch.tensor(seq[[0]], device="cuda"), cb, 0.0, L=L, k=2, V=1)
    assert torch.isnan(soft0).all() and torch.isnan(logZ0).all()


def test_return_internals_is_differentiable(bcjr_mod, oracle):
    _say("return_internals autograd")
    L, N, B = 10, 32, 3
    cb = bcjr_mod.make_3inst_codebook(L, "cuda")
    x = torch.randn(B, N, 1, device="cuda", generator=torch.Generator("cuda").manual_seed(4), requires_grad=True)
    g = torch.randn(B, N, 1, device="cuda", generator=torch.Generator("cuda").manual_seed(5))
    gz = torch.randn(B, device="cuda", generator=torch.Generator("cuda").manual_seed(6))
    soft, logZ, P, la, lb = bcjr_mod.bcjr_forward_backward(x, cb, 0.3, L=L, k=2, V=1, return_internals=True)
    assert soft.requires_grad and logZ.requires_grad and not P.requires_grad
    ((soft * g).sum() + (logZ * gz).sum()).backward()
    x2 = x.detach().clone().requires_grad_(True)
    s2, z2 = bcjr_mod.bcjr_forward_backward(x2, cb, 0.3, L=L, k=2, V=1)
    ((s2 * g).sum() + (z2 * gz).sum()).backward()
    assert torch.equal(soft.detach(), s2.detach()) and torch.equal(logZ.detach(), z2.detach())
    assert torch.equal(x.grad, x2.grad)
    d_ref = oracle.bcjr_backward(x.detach().cpu().numpy(), cb.cpu().numpy(), 0.3, L, 2, g.cpu().numpy(),
                                 gz.cpu().numpy())
    assert max_rel(x.grad.cpu().numpy(), d_ref) < GRAD_TOL


def test_python_float_T_graph_capture(bcjr_mod):
    """A python-float T inside a captured graph: replays match eager, with eager
    work and other temperatures used between replays."""
    _say("graph capture, float T")
    L, B, N = 12, 16, 128
    cb = bcjr_mod.make_1mad_codebook(L, "cuda")
    x = torch.randn(B, N, 1, device="cuda", generator=torch.Generator("cuda").manual_seed(7), requires_grad=True)
    g = torch.randn(B, N, 1, device="cuda", generator=torch.Generator("cuda").manual_seed(8))
    soft, _ = bcjr_mod.bcjr_forward_backward(x, cb, 0.15, L=L, k=2, V=1)
    soft.backward(g)
    ref_soft, ref_grad = soft.detach().clone(), x.grad.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        xg = x.detach().clone().requires_grad_(True)
        for _ in range(2):
            xg.grad = None
            out, _ = bcjr_mod.bcjr_forward_backward(xg, cb, 0.15, L=L, k=2, V=1)
            out.backward(g)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    xg.grad = None
    with torch.cuda.graph(graph):
        out, _ = bcjr_mod.bcjr_forward_backward(xg, cb, 0.15, L=L, k=2, V=1)
        out.backward(g)
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.detach(), ref_soft), i
        assert torch.equal(xg.grad, ref_grad), i
        other, _ = bcjr_mod.bcjr_forward_backward(x.detach(), cb, 0.05 + 0.1 * i, L=L, k=2, V=1)
        _ = float(other.sum())


def test_unseen_table_inside_a_capture_warns_and_runs_the_table_kernels(bcjr_mod, oracle):
    """A 3INST table made without the generator tag and first seen inside a
    graph capture cannot be recognised there (no read-back): the node warns once
    and runs the table kernels, whose replays still match the oracle."""
    _say("unseen table under capture")
    L, B, N, T = 12, 8, 64, 0.2
    plain = bcjr_mod.make_3inst_codebook(L, "cuda").clone()
    assert not hasattr(plain, "_bcjr_code")
    x = torch.randn(B, N, 1, device="cuda", generator=torch.Generator("cuda").manual_seed(11))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with pytest.warns(RuntimeWarning, match="table kernels"):
        with torch.cuda.stream(s):
            with torch.cuda.graph(graph):
                out, _ = bcjr_mod.bcjr_forward_backward(x, plain, T, L=L, k=2, V=1)
    torch.cuda.current_stream().wait_stream(s)
    s_ref, _ = oracle.bcjr_forward(x.cpu().numpy(), plain.cpu().numpy(), T, L, 2)
    for i in range(2):
        graph.replay()
        torch.cuda.synchronize()
        assert max_rel(out.cpu().numpy(), s_ref) < SOFT_TOL, i


def test_torch_compile_fullgraph_quantize_weight(bcjr_mod):
    """torch.compile(fullgraph=True) over bcjr_quantize_weight: no graph break;
    values and gradients equal the eager call's (the same kernels run)."""
    _say("torch.compile fullgraph")
    import torch._dynamo
    from bcjr import bcjr_quantize_weight, make_sign_vector
    L = 12
    cb = bcjr_mod.make_3inst_codebook(L, "cuda")
    m, n = 128, 64
    W0 = torch.randn(m, n, device="cuda", generator=torch.Generator("cuda").manual_seed(9))
    sl = torch.tensor(make_sign_vector(m, 1), device="cuda")
    sr = torch.tensor(make_sign_vector(n, 2), device="cuda")
    T = torch.tensor(0.2, device="cuda")
    G = torch.randn(m, n, device="cuda", generator=torch.Generator("cuda").manual_seed(10))

    def f(W):
        return bcjr_quantize_weight(W, sl, sr, cb, T, L=L, k=2, V=1)

    torch._dynamo.reset()
    cf = torch.compile(f, fullgraph=True, backend="aot_eager")
    outs = []
    for fn in (f, cf):
        W = W0.clone().requires_grad_(True)
        Wq = fn(W)
        (Wq * G).sum().backward()
        outs.append((Wq.detach(), W.grad))
    assert max_rel(outs[1][0].cpu().numpy(), outs[0][0].cpu().numpy()) < 1e-6
    assert max_rel(outs[1][1].cpu().numpy(), outs[0][1].cpu().numpy()) < 1e-6


def test_forget_after_writes_that_bypass_the_version_counter(bcjr_mod):
    """A table recognised as 3INST and then changed through .data (no version
    bump) keeps its cached recognition until forget(); afterwards it is examined
    afresh and runs on the table kernels."""
    _say("forget")
    from bcjr import ops
    from bcjr.codes import forget, resolve_codebook
    dev = torch.device("cuda")
    L = 12
    plain = bcjr_mod.make_3inst_codebook(L, dev).clone()
    assert resolve_codebook(plain, L, 2, 1, dev)[0].code == ops.CODE_3INST
    plain.data[7, 0] += 1.0  # bypasses the version counter
    assert resolve_codebook(plain, L, 2, 1, dev)[0].code == ops.CODE_3INST  # stale by design
    forget(plain)
    spec, table = resolve_codebook(plain, L, 2, 1, dev)
    assert spec.code == ops.CODE_TABLE and table.data_ptr() == plain.data_ptr()


def test_numpy_api_reuses_device_tables_by_content(bcjr_mod):
    """viterbi_encode_v builds its device table from decode_fn on each call; an
    identical table reuses one device tensor (its recognition cached), and a
    decode_fn whose table changed in place gets a fresh one."""
    _say("numpy-api table cache")
    from bcjr import encode
    L, V = 10, 2
    lut = np.random.default_rng(4).standard_normal((1 << L, V)).astype(np.float32)

    def decode(states):
        return lut[states]

    a = encode._gpu_codebook(L, V, decode)
    b = encode._gpu_codebook(L, V, decode)
    assert a is b
    lut[3] += 1.0
    c = encode._gpu_codebook(L, V, decode)
    assert c is not a and np.array_equal(c.cpu().numpy(), lut)
    seq = np.random.default_rng(5).standard_normal(64).astype(np.float32)
    r1 = bcjr_mod.viterbi_encode_v(seq, L, 1, V, decode)
    r2 = bcjr_mod.viterbi_encode_v(seq, L, 1, V, decode)
    assert np.array_equal(r1[0], r2[0]) and r1[1] == r2[1]
