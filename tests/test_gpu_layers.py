"""GroupCDL-style layers (circulant_attention.layers) on the GPU against
float64 CPU compositions of the oracle.

* CircAttBlock: x + W_o MHA(W_q x, W_k x, W_v x), channels-last, fused
  attention.  Reference: the oracle's attention forward / backward
  (src/attention.jl:38-42 with the rrules of src/rrules.jl) and the linear
  maps' chain rule in numpy; values within 1e-5, gradients within 1e-4.
* GroupThresholding: z relu(1 - tau / sqrt(Γ ⨷ z² + eps)) with Γ the
  circulant_mh_adjacency of θ = W_θ f.  Reference forward from the oracle's
  similarity, softmax and apply; gradients (z, f, W_θ, tau) checked as
  directional derivatives against central differences of that float64
  forward.  The fused and materialised forms are compared with each other.
"""
import numpy as np
import pytest

from conftest import TOL_FWD, TOL_GRAD, rel_err

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import oracle as O  # noqa: E402


def host(t):
    return t.detach().cpu().double().numpy()


def to_planar(a):
    """numpy (B, *spatial, C) -> (B, C, *spatial)."""
    return np.ascontiguousarray(np.moveaxis(a, -1, 1))


def to_cl(a):
    return np.ascontiguousarray(np.moveaxis(a, 1, -1))


@pytest.mark.parametrize("kind", [0, 1], ids=["dot", "dist"])
@pytest.mark.parametrize("shape,nheads,ws", [((2, 14, 18, 32), 2, 7), ((1, 20, 16, 16), 1, 15),
                                             ((2, 60, 32), 2, 9)],
                         ids=["2d-nh2-ws7", "2d-nh1-ws15", "1d-nh2-ws9"])
def test_circattblock_matches_reference(cuda, kind, shape, nheads, ws):
    import circulant_attention as ca

    torch.manual_seed(3)
    C = shape[-1]
    simfun = ca.DistanceSimilarity() if kind else ca.DotSimilarity()
    blk = ca.CircAttBlock(C, ws, nheads, simfun).to(cuda)
    x = torch.randn(shape, device=cuda, requires_grad=True)
    w = torch.randn(shape, device=cuda)
    out = blk(x)
    (out * w).sum().backward()

    W = {n: host(getattr(blk, n).weight) for n in "qkvo"}
    b = {n: host(getattr(blk, n).bias) for n in "qkvo"}
    xh, wh = host(x), host(w)
    q, k, v = (xh @ W[n].T + b[n] for n in "qkv")
    y, A = O.attention_fwd(kind, to_planar(q), to_planar(k), to_planar(v), ws, nheads)
    y = to_cl(y)
    ref = xh + y @ W["o"].T + b["o"]
    assert rel_err(host(out), ref) < TOL_FWD
    dy = wh @ W["o"]
    dq, dk, dv = (to_cl(t) for t in O.attention_bwd(kind, to_planar(q), to_planar(k), to_planar(v),
                                                     to_planar(dy), ws, nheads, A=A))
    dx = wh + dq @ W["q"] + dk @ W["k"] + dv @ W["v"]
    flat = lambda a: a.reshape(-1, a.shape[-1])
    ref_grads = {"x": dx,
                 "o.weight": flat(wh).T @ flat(y), "o.bias": flat(wh).sum(0),
                 "q.weight": flat(dq).T @ flat(xh), "q.bias": flat(dq).sum(0),
                 "k.weight": flat(dk).T @ flat(xh), "k.bias": flat(dk).sum(0),
                 "v.weight": flat(dv).T @ flat(xh), "v.bias": flat(dv).sum(0)}
    got = {"x": host(x.grad)}
    for n, p in blk.named_parameters():
        got[n] = host(p.grad)
    for n, r in ref_grads.items():
        if n == "k.bias" and kind == 0:
            # q.(k_j + b) shifts every score of a row by q.b, which the
            # softmax ignores: the exact gradient is zero; measure against
            # the query bias's scale instead
            err = np.abs(got[n] - r).max() / np.abs(ref_grads["q.bias"]).max()
        else:
            err = rel_err(got[n], r)
        assert err < TOL_GRAD, (n, err)


def group_threshold_ref(kind, z, f, Wt, tau, ws, nheads, eps):
    """float64 forward of GroupThresholding from the oracle's pieces."""
    th = to_planar(f @ Wt.T)
    zp = to_planar(z)
    dims = O.spatial_dims(th)
    K = ws ** len(dims)
    thf, z2f = O._flat(th, nheads), O._flat(zp * zp, nheads)
    S = O.similarity(kind, thf, thf, dims, ws, 1.0)
    A = O.softmax(S, K)
    xi = to_cl(O.apply(A, z2f, dims, ws).reshape(zp.shape))
    return z * np.maximum(1.0 - tau / np.sqrt(xi + eps), 0.0)


@pytest.mark.parametrize("fused", [True, False], ids=["fused", "materialised"])
@pytest.mark.parametrize("kind", [0, 1], ids=["dot", "dist"])
def test_group_thresholding_matches_reference(cuda, kind, fused):
    import circulant_attention as ca

    torch.manual_seed(7)
    B, H, Wd, M, F, nheads, ws, eps = 2, 12, 16, 32, 24, 2, 7, 1e-6
    simfun = ca.DistanceSimilarity() if kind else ca.DotSimilarity()
    gt = ca.GroupThresholding(M, F, ws, nheads, simfun, tau=0.3, eps=eps, fused=fused).to(cuda)
    with torch.no_grad():
        gt.theta.weight.mul_(0.5)
        gt.tau.copy_(0.3 + 0.1 * torch.rand(M, device=cuda))
    z = torch.randn((B, H, Wd, M), device=cuda, requires_grad=True)
    f = torch.randn((B, H, Wd, F), device=cuda, requires_grad=True)
    w = torch.randn((B, H, Wd, M), device=cuda)
    out = gt(z, f)
    (out * w).sum().backward()

    zh, fh, wh = host(z), host(f), host(w)
    Wt, tau = host(gt.theta.weight), host(gt.tau)
    ref = group_threshold_ref(kind, zh, fh, Wt, tau, ws, nheads, eps)
    assert rel_err(host(out), ref) < TOL_FWD

    loss = lambda z_, f_, W_, t_: float((group_threshold_ref(kind, z_, f_, W_, t_, ws, nheads, eps)
                                         * wh).sum())
    grads = {"z": host(z.grad), "f": host(f.grad), "W": host(gt.theta.weight.grad),
             "tau": host(gt.tau.grad)}
    rng = np.random.default_rng(1)
    base = {"z": zh, "f": fh, "W": Wt, "tau": tau}
    h = 1e-5
    for name in ("z", "f", "W", "tau"):
        for _ in range(2):
            u = rng.standard_normal(base[name].shape)
            args_p = dict(base)
            args_m = dict(base)
            args_p[name] = base[name] + h * u
            args_m[name] = base[name] - h * u
            fd = (loss(args_p["z"], args_p["f"], args_p["W"], args_p["tau"]) -
                  loss(args_m["z"], args_m["f"], args_m["W"], args_m["tau"])) / (2 * h)
            g = float((grads[name] * u).sum())
            bound = TOL_GRAD * (np.linalg.norm(grads[name]) * np.linalg.norm(u) + abs(fd))
            assert abs(g - fd) <= bound, (name, g, fd)


def test_group_thresholding_reuses_an_adjacency(cuda):
    """forward(z, A=adjacency(f)) equals forward(z, f) in both forms."""
    import circulant_attention as ca

    torch.manual_seed(9)
    gt = ca.GroupThresholding(16, 16, 5, 2, ca.DistanceSimilarity(), fused=True).to(cuda)
    z = torch.randn((1, 10, 12, 16), device=cuda)
    f = torch.randn((1, 10, 12, 16), device=cuda)
    with torch.no_grad():
        A = gt.adjacency(f)
        a = gt(z, A=A)
        b = gt(z, f)
    assert rel_err(host(a), host(b)) < TOL_FWD
