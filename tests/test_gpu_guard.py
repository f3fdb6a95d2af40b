"""Reads and writes outside a kernel's tensors, tested from outside (GPU).

Every tensor handed to an entry point here sits inside a larger buffer. The elements
around it (a band before it, a band after it, and the padding between rows where the
row stride exceeds the row) hold a NaN bit pattern of the tensor's dtype, and so do an
output's own elements before the call. A kernel that reads an element outside its
tensor and uses it returns a result different from the same call on tightly packed
tensors (compared bit for bit); a kernel that writes outside its output changes the
pattern; a kernel that leaves an output element unwritten leaves NaN there. Shapes are
ragged: rows and sizes that are not multiples of the 16-byte vector (the tail and
element-wise paths), row strides that are not, widths on either side of the register
plans' limits, and the vocabulary and hidden sizes of the linear CE's masked tails.
"""
import ctypes

import pytest
import torch

from helpers import G, GUARD_BITS as _BITS, Guarded, flat, same
from trainscale_amd import _lib, ops

pytestmark = pytest.mark.gpu
BF, F16, F32 = torch.bfloat16, torch.float16, torch.float32
P = ctypes.c_void_p


def code(dtype):
    return _lib.DTYPE_CODE[dtype]


def st(dev):
    return _lib.stream_handle(dev)


def ok(status, what):
    _lib.check(status, what)


# ---------------------------------------------------------------------------
# RMSNorm forward, backward, fused add
# ---------------------------------------------------------------------------

RMS_SHAPES = [(37, 4096, 8, BF), (5, 256, 8, BF), (300, 1000, 24, BF), (33, 1001, 3, BF),
              (64, 2048, 8, BF), (65, 1024, 16, BF), (3, 520, 8, BF), (17, 8192, 8, BF),
              (7, 72, 8, F32), (129, 520, 8, F16), (9, 4100, 4, F32)]


@pytest.mark.parametrize("rows,cols,pad,dtype", RMS_SHAPES)
def test_rmsnorm_stays_inside(gpu, rows, cols, pad, dtype):
    lib = _lib.load()
    g = torch.Generator(device=gpu).manual_seed(rows * cols)
    x = torch.randn(rows, cols, device=gpu, generator=g).to(dtype)
    dy = torch.randn(rows, cols, device=gpu, generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(cols, device=gpu, generator=g)).to(dtype)
    ld = cols + pad
    eps = 1e-6
    # packed reference calls
    y0 = torch.empty_like(x)
    r0 = torch.empty(rows, device=gpu)
    ok(lib.ts_rmsnorm_fwd(P(x.data_ptr()), cols, code(dtype), P(w.data_ptr()), code(dtype),
                          P(y0.data_ptr()), cols, P(r0.data_ptr()), rows, cols, eps, 0, st(gpu)),
       "fwd")
    wsb = int(lib.ts_rmsnorm_bwd_workspace_size(rows, cols))
    ws0 = torch.empty(max(wsb, 1), dtype=torch.uint8, device=gpu)
    dx0 = torch.empty_like(x)
    dw0 = torch.empty_like(w)
    ok(lib.ts_rmsnorm_bwd(P(dy.data_ptr()), cols, P(x.data_ptr()), cols, code(dtype),
                          P(w.data_ptr()), code(dtype), P(r0.data_ptr()), P(dx0.data_ptr()), cols,
                          P(dw0.data_ptr()), P(ws0.data_ptr()), wsb, rows, cols, st(gpu)), "bwd")
    # the same calls inside guard bands, strided rows in and out
    gx = Guarded(rows, cols, ld, dtype, gpu, x)
    gdy = Guarded(rows, cols, ld + 8, dtype, gpu, dy)
    gw = flat(cols, dtype, gpu, w)
    gy = Guarded(rows, cols, ld, dtype, gpu)
    gr = flat(rows, F32, gpu)
    ok(lib.ts_rmsnorm_fwd(gx.p, ld, code(dtype), gw.p, code(dtype), gy.p, ld, gr.p, rows, cols,
                          eps, 0, st(gpu)), "fwd guarded")
    gdx = Guarded(rows, cols, ld, dtype, gpu)
    gdw = flat(cols, dtype, gpu)
    gws = flat(max(wsb, 1), torch.uint8, gpu)
    ok(lib.ts_rmsnorm_bwd(gdy.p, ld + 8, gx.p, ld, code(dtype), gw.p, code(dtype), gr.p, gdx.p,
                          ld, gdw.p, gws.p, wsb, rows, cols, st(gpu)), "bwd guarded")
    torch.cuda.synchronize()
    assert same(gy.t, y0) and same(gr.t[0], r0)
    assert same(gdx.t, dx0) and same(gdw.t[0], dw0)
    for name, t in (("x", gx), ("dy", gdy), ("w", gw), ("y", gy), ("rstd", gr), ("dx", gdx),
                    ("dw", gdw), ("workspace", gws)):
        assert t.intact(), f"{name}: a write outside the tensor"


@pytest.mark.parametrize("rows,cols,pad,dtype", [(37, 4096, 8, BF), (33, 1001, 3, BF),
                                                 (5, 256, 8, F16), (7, 72, 4, F32),
                                                 (300, 1000, 24, BF)])
def test_add_rmsnorm_stays_inside(gpu, rows, cols, pad, dtype):
    lib = _lib.load()
    g = torch.Generator(device=gpu).manual_seed(rows + cols)
    x = torch.randn(rows, cols, device=gpu, generator=g).to(dtype)
    r = torch.randn(rows, cols, device=gpu, generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(cols, device=gpu, generator=g)).to(dtype)
    y0, h0 = torch.empty_like(x), torch.empty_like(x)
    s0 = torch.empty(rows, device=gpu)
    ok(lib.ts_add_rmsnorm_fwd(P(x.data_ptr()), cols, P(r.data_ptr()), cols, code(dtype),
                              P(w.data_ptr()), code(dtype), P(y0.data_ptr()), cols,
                              P(h0.data_ptr()), cols, P(s0.data_ptr()), rows, cols, 1e-6, 1,
                              st(gpu)), "add")
    # strides that keep the packed call's path (whole 16-byte vectors per row where the
    # row is), so both calls sum the squares in the same order
    ld = cols + pad
    ld2 = ld + pad
    gx, gr_ = Guarded(rows, cols, ld, dtype, gpu, x), Guarded(rows, cols, ld2, dtype, gpu, r)
    gw = flat(cols, dtype, gpu, w)
    gy, gh = Guarded(rows, cols, ld, dtype, gpu), Guarded(rows, cols, ld2, dtype, gpu)
    gs = flat(rows, F32, gpu)
    ok(lib.ts_add_rmsnorm_fwd(gx.p, ld, gr_.p, ld2, code(dtype), gw.p, code(dtype), gy.p, ld,
                              gh.p, ld2, gs.p, rows, cols, 1e-6, 1, st(gpu)), "add guarded")
    torch.cuda.synchronize()
    assert same(gy.t, y0) and same(gh.t, h0) and same(gs.t[0], s0)
    for t in (gx, gr_, gw, gy, gh, gs):
        assert t.intact()


# ---------------------------------------------------------------------------
# RoPE (tables and in-register angles, forward and backward)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("B,S,Hq,Hk,D,il,dtype", [
    (2, 37, 32, 8, 128, False, BF), (1, 64, 3, 1, 64, True, BF), (3, 9, 2, 2, 20, False, F32),
    (2, 17, 8, 8, 256, False, F16), (1, 5, 40, 8, 128, True, BF)])
@pytest.mark.parametrize("mode", ["table", "register"])
def test_rope_stays_inside(gpu, B, S, Hq, Hk, D, il, dtype, mode):
    import oracle
    g = torch.Generator(device=gpu).manual_seed(S * D + Hq)
    q = torch.randn(B, S, Hq, D, device=gpu, generator=g).to(dtype)
    k = torch.randn(B, S, Hk, D, device=gpu, generator=g).to(dtype)
    pos = torch.stack([torch.randperm(S) for _ in range(B)]).to(gpu)
    cos, sin = oracle.rope_tables(D, S, 10000.0)
    inv = 1.0 / (10000.0 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    kw = (dict(cos=cos.to(gpu), sin=sin.to(gpu)) if mode == "table" else dict(inv_freq=inv))
    for backward in (False, True):
        q0, k0 = torch.empty_like(q), torch.empty_like(k)
        ops.rope_apply(q, q0, k, k0, position_ids=pos, interleaved=il, backward=backward, **kw)
        # token rows of Hq * D (Hk * D) elements with a padded stride, inside guard bands
        gq = Guarded(B * S, Hq * D, Hq * D + 8, dtype, gpu, q)
        gk = Guarded(B * S, Hk * D, Hk * D + 24, dtype, gpu, k)
        gqo = Guarded(B * S, Hq * D, Hq * D + 16, dtype, gpu)
        gko = Guarded(B * S, Hk * D, Hk * D + 8, dtype, gpu)
        view = lambda t, h: t.t.view(B, S, h, D)
        ops.rope_apply(view(gq, Hq), view(gqo, Hq), view(gk, Hk), view(gko, Hk),
                       position_ids=pos, interleaved=il, backward=backward, **kw)
        torch.cuda.synchronize()
        assert same(gqo.t, q0.reshape(B * S, -1)) and same(gko.t, k0.reshape(B * S, -1))
        for t in (gq, gk, gqo, gko):
            assert t.intact()


# ---------------------------------------------------------------------------
# Cross-entropy: one-pass (schedule B), forward then backward (schedule A)
# ---------------------------------------------------------------------------

CE_SHAPES = [(40, 50257, 7, BF), (33, 32000, 8, BF), (17, 1000, 8, F16), (9, 4096, 8, F32),
             (3, 140000, 8, BF), (12, 131072, 8, BF), (5, 77, 3, BF)]


def _labels(N, V, gpu):
    g = torch.Generator().manual_seed(N * 7 + V)
    lab = torch.randint(0, V, (N,), generator=g)
    lab[::4] = -100
    return lab.to(gpu)


@pytest.mark.parametrize("N,V,pad,dtype", CE_SHAPES)
def test_ce_one_pass_stays_inside(gpu, N, V, pad, dtype):
    lib = _lib.load()
    logits = (2 * torch.randn(N, V, device=gpu, generator=torch.Generator(device=gpu)
                              .manual_seed(N + V))).to(dtype)
    lab = _labels(N, V, gpu)
    dl = torch.full((1,), 0.37, device=gpu)
    l0, s0, gr0 = torch.empty(N, device=gpu), torch.empty(N, device=gpu), torch.empty_like(logits)
    ok(lib.ts_ce_fwd_bwd(P(logits.data_ptr()), V, code(dtype), P(lab.data_ptr()), N, V, -100,
                         0.0, 0.0, 0.0, P(dl.data_ptr()), 0, 1.0, P(l0.data_ptr()),
                         P(s0.data_ptr()), P(gr0.data_ptr()), V, code(dtype), st(gpu)), "ce")
    gl = Guarded(N, V, V + pad, dtype, gpu, logits)
    gloss, glse = flat(N, F32, gpu), flat(N, F32, gpu)
    ggrad = Guarded(N, V, V + pad + 8, dtype, gpu)
    ok(lib.ts_ce_fwd_bwd(gl.p, V + pad, code(dtype), P(lab.data_ptr()), N, V, -100, 0.0, 0.0,
                         0.0, P(dl.data_ptr()), 0, 1.0, gloss.p, glse.p, ggrad.p, V + pad + 8,
                         code(dtype), st(gpu)), "ce guarded")
    torch.cuda.synchronize()
    assert same(gloss.t[0], l0) and same(glse.t[0], s0) and same(ggrad.t, gr0)
    for t in (gl, gloss, glse, ggrad):
        assert t.intact()


@pytest.mark.parametrize("N,V,pad,dtype", CE_SHAPES)
def test_ce_two_pass_stays_inside(gpu, N, V, pad, dtype):
    lib = _lib.load()
    logits = (2 * torch.randn(N, V, device=gpu, generator=torch.Generator(device=gpu)
                              .manual_seed(N * V))).to(dtype)
    lab = _labels(N, V, gpu)
    dl = (0.1 + torch.rand(N, device=gpu)).contiguous()
    l0, s0, gr0 = torch.empty(N, device=gpu), torch.empty(N, device=gpu), torch.empty_like(logits)
    ok(lib.ts_ce_fwd(P(logits.data_ptr()), V, code(dtype), P(lab.data_ptr()), N, V, -100, 0.8,
                     25.0, 0.0, P(l0.data_ptr()), P(s0.data_ptr()), st(gpu)), "fwd")
    ok(lib.ts_ce_bwd(P(logits.data_ptr()), V, code(dtype), P(lab.data_ptr()), P(s0.data_ptr()),
                     P(dl.data_ptr()), 1, 1.0, P(gr0.data_ptr()), V, code(dtype), N, V, -100,
                     0.8, 25.0, 0.0, st(gpu)), "bwd")
    gl = Guarded(N, V, V + pad, dtype, gpu, logits)
    gloss, glse = flat(N, F32, gpu), flat(N, F32, gpu)
    ggrad = Guarded(N, V, V + pad + 16, dtype, gpu)
    ok(lib.ts_ce_fwd(gl.p, V + pad, code(dtype), P(lab.data_ptr()), N, V, -100, 0.8, 25.0, 0.0,
                     gloss.p, glse.p, st(gpu)), "fwd guarded")
    ok(lib.ts_ce_bwd(gl.p, V + pad, code(dtype), P(lab.data_ptr()), glse.p, P(dl.data_ptr()), 1,
                     1.0, ggrad.p, V + pad + 16, code(dtype), N, V, -100, 0.8, 25.0, 0.0,
                     st(gpu)), "bwd guarded")
    torch.cuda.synchronize()
    assert same(gloss.t[0], l0) and same(glse.t[0], s0) and same(ggrad.t, gr0)
    for t in (gl, gloss, glse, ggrad):
        assert t.intact()


@pytest.mark.parametrize("N,Vp,pad,dtype", [(40, 16032, 8, BF), (17, 6283, 5, BF),
                                            (9, 1000, 8, F32)])
def test_vocab_shard_stays_inside(gpu, N, Vp, pad, dtype):
    lib = _lib.load()
    x = torch.randn(N, Vp, device=gpu).to(dtype)
    t = _labels(N, 3 * Vp, gpu)
    v0 = Vp
    s0 = torch.empty(N, 4, device=gpu)
    ok(lib.ts_ce_vocab_shard_stats(P(x.data_ptr()), Vp, code(dtype), P(t.data_ptr()), N, Vp, v0,
                                   P(s0.data_ptr()), st(gpu)), "stats")
    gx = Guarded(N, Vp, Vp + pad, dtype, gpu, x)
    gs = flat(N * 4, F32, gpu)
    ok(lib.ts_ce_vocab_shard_stats(gx.p, Vp + pad, code(dtype), P(t.data_ptr()), N, Vp, v0,
                                   gs.p, st(gpu)), "stats guarded")
    lse = torch.logsumexp(torch.cat([x.float(), x.float() + 0.5], 1), 1).contiguous()
    go = torch.ones(1, device=gpu)
    g0 = torch.empty_like(x)
    ok(lib.ts_ce_vocab_shard_bwd(P(x.data_ptr()), Vp, code(dtype), P(t.data_ptr()),
                                 P(lse.data_ptr()), P(go.data_ptr()), 1.0 / N, N, Vp, v0, 0.1,
                                 P(g0.data_ptr()), Vp, code(dtype), st(gpu)), "bwd")
    gg = Guarded(N, Vp, Vp + pad + 8, dtype, gpu)
    ok(lib.ts_ce_vocab_shard_bwd(gx.p, Vp + pad, code(dtype), P(t.data_ptr()), P(lse.data_ptr()),
                                 P(go.data_ptr()), 1.0 / N, N, Vp, v0, 0.1, gg.p, Vp + pad + 8,
                                 code(dtype), st(gpu)), "bwd guarded")
    torch.cuda.synchronize()
    assert same(gs.t[0], s0.reshape(-1)) and same(gg.t, g0)
    for g in (gx, gs, gg):
        assert g.intact()


# ---------------------------------------------------------------------------
# SwiGLU and the in-place scale (element counts that are not whole vectors)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("n,dtype", [(1000003, BF), (4096 * 7 + 5, F16), (77, F32), (8, BF)])
def test_swiglu_and_scale_stay_inside(gpu, n, dtype):
    lib = _lib.load()
    gate = torch.randn(n, device=gpu).to(dtype)
    up = torch.randn(n, device=gpu).to(dtype)
    dout = torch.randn(n, device=gpu).to(dtype)
    o0, dg0, du0 = torch.empty_like(gate), torch.empty_like(gate), torch.empty_like(gate)
    ok(lib.ts_swiglu_fwd(P(gate.data_ptr()), P(up.data_ptr()), P(o0.data_ptr()), n, code(dtype),
                         st(gpu)), "fwd")
    ok(lib.ts_swiglu_bwd(P(dout.data_ptr()), P(gate.data_ptr()), P(up.data_ptr()),
                         P(dg0.data_ptr()), P(du0.data_ptr()), n, code(dtype), st(gpu)), "bwd")
    gg, gu, gd = flat(n, dtype, gpu, gate), flat(n, dtype, gpu, up), flat(n, dtype, gpu, dout)
    go, gdg, gdu = flat(n, dtype, gpu), flat(n, dtype, gpu), flat(n, dtype, gpu)
    ok(lib.ts_swiglu_fwd(gg.p, gu.p, go.p, n, code(dtype), st(gpu)), "fwd guarded")
    ok(lib.ts_swiglu_bwd(gd.p, gg.p, gu.p, gdg.p, gdu.p, n, code(dtype), st(gpu)), "bwd guarded")
    # the scale in place, 16-byte aligned and not (one element in)
    two = torch.full((1,), 2.5, device=gpu)
    s0 = o0.clone()
    ok(lib.ts_scale_inplace(P(s0.data_ptr()), n, code(dtype), P(two.data_ptr()), st(gpu)), "s")
    gs = flat(n, dtype, gpu, o0)
    ok(lib.ts_scale_inplace(gs.p, n, code(dtype), P(two.data_ptr()), st(gpu)), "s guarded")
    m = n - 1
    s1 = o0[1:].clone()
    ok(lib.ts_scale_inplace(P(s1.data_ptr()), m, code(dtype), P(two.data_ptr()), st(gpu)), "s1")
    gs1 = flat(m, dtype, gpu, o0[1:])
    gs1.t = gs1.buf[G + 1:G + 1 + m].view(1, m)  # one element further: not 16-byte aligned
    gs1.t.copy_(o0[1:].reshape(1, m))
    gs1.buf[G].view(_BITS[dtype][0]).fill_(_BITS[dtype][1])
    ok(lib.ts_scale_inplace(P(gs1.t.data_ptr()), m, code(dtype), P(two.data_ptr()), st(gpu)),
       "s1 guarded")
    torch.cuda.synchronize()
    assert same(go.t[0], o0) and same(gdg.t[0], dg0) and same(gdu.t[0], du0)
    assert same(gs.t[0], s0) and same(gs1.t[0], s1)
    for g in (gg, gu, gd, go, gdg, gdu, gs):
        assert g.intact()
    iv, bits = _BITS[dtype]
    rest = torch.cat([gs1.buf[:G + 1], gs1.buf[G + 1 + m:]])
    assert bool((rest.view(iv) == bits).all())


# ---------------------------------------------------------------------------
# Fused linear CE: one call in token chunks, two-pass, kept logits, vocabulary shard
# ---------------------------------------------------------------------------

LCE_SHAPES = [(264, 256, 1001, 8, 256), (520, 128, 50257, 16, 256), (136, 104, 777, 8, 0),
              (1032, 64, 4096, 24, 512)]


def _lce_inputs(N, H, V, gpu):
    g = torch.Generator(device=gpu).manual_seed(N + H + V)
    h = torch.randn(N, H, device=gpu, generator=g).to(BF)
    w = (0.05 * torch.randn(V, H, device=gpu, generator=g)).to(BF)
    lab = _labels(N, V, gpu)
    return h, w, lab


@pytest.mark.parametrize("N,H,V,pad,chunk", LCE_SHAPES)
@pytest.mark.parametrize("flags", [1, 3])
def test_linear_ce_one_call_stays_inside(gpu, N, H, V, pad, chunk, flags):
    lib = _lib.load()
    h, w, lab = _lce_inputs(N, H, V, gpu)
    wsb = int(lib.ts_flce_workspace_size(N, H, V, chunk, flags))
    outs = []
    for guarded in (False, True):
        if guarded:
            gh_in, gw_in = Guarded(N, H, H + pad, BF, gpu, h), Guarded(V, H, H + pad + 8, BF, gpu, w)
            hp, ldh, wp, ldw = gh_in.p, H + pad, gw_in.p, H + pad + 8
        else:
            hp, ldh, wp, ldw = P(h.data_ptr()), H, P(w.data_ptr()), H
        loss, rows, lse = flat(1, F32, gpu), flat(N, F32, gpu), flat(N, F32, gpu)
        gh, gw = Guarded(N, H, H, BF, gpu), Guarded(V, H, H, BF, gpu)
        ws = flat(max(wsb, 1), torch.uint8, gpu)
        ok(lib.ts_flce_fwd_bwd(hp, ldh, wp, ldw, P(lab.data_ptr()), N, H, V, -100, 0, loss.p,
                               rows.p, lse.p, gh.p, gw.p, chunk, flags & 2, ws.p, wsb, st(gpu)),
           "flce")
        torch.cuda.synchronize()
        bufs = [loss, rows, lse, gh, gw, ws] + ([gh_in, gw_in] if guarded else [])
        for b in bufs:
            assert b.intact(), "a write outside the tensor"
        outs.append([loss.t, rows.t, lse.t, gh.t, gw.t])
    for a, b in zip(*outs):
        assert same(a, b)


@pytest.mark.parametrize("N,H,V,pad,chunk", LCE_SHAPES)
def test_linear_ce_two_pass_and_kept_stay_inside(gpu, N, H, V, pad, chunk):
    lib = _lib.load()
    h, w, lab = _lce_inputs(N, H, V, gpu)
    dl = (0.5 + torch.rand(N, device=gpu)).contiguous()
    wf = int(lib.ts_flce_forward_workspace_size(N, V))
    wb = int(lib.ts_flce_backward_workspace_size(N, H, V, 512))
    wk = int(lib.ts_flce_backward_kept_workspace_size(N))
    ldl = -(-V // 8) * 8
    outs = []
    for guarded in (False, True):
        if guarded:
            gh_in, gw_in = Guarded(N, H, H + pad, BF, gpu, h), Guarded(V, H, H + pad + 8, BF, gpu, w)
            hp, ldh, wp, ldw = gh_in.p, H + pad, gw_in.p, H + pad + 8
        else:
            hp, ldh, wp, ldw = P(h.data_ptr()), H, P(w.data_ptr()), H
        rows, lse = flat(N, F32, gpu), flat(N, F32, gpu)
        wsf, wsb_, wsk = (flat(max(wf, 1), torch.uint8, gpu), flat(max(wb, 1), torch.uint8, gpu),
                          flat(max(wk, 1), torch.uint8, gpu))
        xf = (3.0, 0.8, 0.7)  # softcap, scale, temperature: the RL form
        ok(lib.ts_flce_forward(hp, ldh, wp, ldw, P(lab.data_ptr()), N, H, V, -100, 2, *xf, None,
                               rows.p, lse.p, wsf.p, wf, st(gpu)), "forward")
        gh, gw = Guarded(N, H, H, BF, gpu), Guarded(V, H, H, BF, gpu)
        ok(lib.ts_flce_backward(hp, ldh, wp, ldw, P(lab.data_ptr()), N, H, V, -100, 2, *xf,
                                lse.p, P(dl.data_ptr()), 1, gh.p, gw.p, 512, wsb_.p, wb, st(gpu)),
           "backward")
        rows2, lse2 = flat(N, F32, gpu), flat(N, F32, gpu)
        kept = Guarded(N, ldl, ldl, BF, gpu)
        ok(lib.ts_flce_forward_keep(hp, ldh, wp, ldw, P(lab.data_ptr()), N, H, V, -100, 2, *xf,
                                    None, rows2.p, lse2.p, kept.p, wsf.p, wf, st(gpu)), "keep")
        gh2, gw2 = Guarded(N, H, H, BF, gpu), Guarded(V, H, H, BF, gpu)
        ok(lib.ts_flce_backward_kept(hp, ldh, wp, ldw, P(lab.data_ptr()), N, H, V, -100, 2, *xf,
                                     lse2.p, P(dl.data_ptr()), 1, kept.p, gh2.p, gw2.p, wsk.p, wk,
                                     st(gpu)), "kept")
        torch.cuda.synchronize()
        bufs = [rows, lse, gh, gw, rows2, lse2, gh2, gw2, kept, wsf, wsb_, wsk]
        bufs += [gh_in, gw_in] if guarded else []
        for b in bufs:
            assert b.intact(), "a write outside the tensor"
        outs.append([rows.t, lse.t, gh.t, gw.t, rows2.t, lse2.t, gh2.t, gw2.t])
    for a, b in zip(*outs):
        assert same(a, b)


@pytest.mark.parametrize("N,H,Vp,pad", [(264, 256, 1001, 8), (520, 128, 6283, 16),
                                        (64, 64, 16032, 8)])
def test_linear_ce_vocab_shard_stays_inside(gpu, N, H, Vp, pad):
    lib = _lib.load()
    h, w, _ = _lce_inputs(N, H, Vp, gpu)
    lab = _labels(N, 3 * Vp, gpu)
    v0 = Vp
    wsb = int(lib.ts_flce_vocab_workspace_size(N, Vp))
    outs = []
    for guarded in (False, True):
        if guarded:
            gh_in, gw_in = Guarded(N, H, H + pad, BF, gpu, h), Guarded(Vp, H, H + pad, BF, gpu, w)
            hp, ldh, wp, ldw = gh_in.p, H + pad, gw_in.p, H + pad
        else:
            hp, ldh, wp, ldw = P(h.data_ptr()), H, P(w.data_ptr()), H
        stats, ws = flat(N * 4, F32, gpu), flat(max(wsb, 1), torch.uint8, gpu)
        ok(lib.ts_flce_vocab_fwd(hp, ldh, wp, ldw, P(lab.data_ptr()), N, H, Vp, v0, stats.p, ws.p,
                                 wsb, st(gpu)), "vocab fwd")
        # three ranks' partials: this one's and two made-up ones
        sa = torch.stack([stats.t[0].view(N, 4) + d for d in (0.0, 0.25, -0.5)]).contiguous()
        loss, rows, lse = flat(1, F32, gpu), flat(N, F32, gpu), flat(N, F32, gpu)
        gh, gw = Guarded(N, H, H, BF, gpu), Guarded(Vp, H, H, BF, gpu)
        ok(lib.ts_flce_vocab_bwd(hp, ldh, wp, ldw, P(lab.data_ptr()), N, H, Vp, v0,
                                 P(sa.data_ptr()), 3, -100, 0, loss.p, rows.p, lse.p, gh.p, gw.p,
                                 ws.p, wsb, st(gpu)), "vocab bwd")
        torch.cuda.synchronize()
        bufs = [stats, ws, loss, rows, lse, gh, gw] + ([gh_in, gw_in] if guarded else [])
        for b in bufs:
            assert b.intact(), "a write outside the tensor"
        outs.append([stats.t, loss.t, rows.t, lse.t, gh.t, gw.t])
    for a, b in zip(*outs):
        assert same(a, b)
