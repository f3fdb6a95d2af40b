"""The C-ABI library loads, exports every declared symbol, and rejects bad calls
on the host before anything reaches a GPU (no compute calls here)."""
import ctypes

import pytest

from trainscale_amd import _lib

TS_OK, INVALID, DTYPE, SHAPE, WORKSPACE = 0, -1, -2, -3, -4
NULL = None


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_every_header_symbol_is_exported(lib):
    names = _lib.header_symbols()
    assert set(names) == set(_lib.SIGNATURES), (names, sorted(_lib.SIGNATURES))
    for name in names:
        assert hasattr(lib, name), name


def test_version_and_error_string(lib):
    assert lib.ts_version().decode().startswith("trainscale_amd")
    assert isinstance(lib.ts_last_error(), bytes)


FAKE = ctypes.c_void_p(0x1000)  # never dereferenced: every call below fails validation


def test_rmsnorm_fwd_validation(lib):
    st = NULL
    assert lib.ts_rmsnorm_fwd(FAKE, 64, 1, FAKE, 1, FAKE, 64, FAKE, -1, 64, 1e-6, 0, st) == SHAPE
    assert lib.ts_rmsnorm_fwd(FAKE, 64, 7, FAKE, 1, FAKE, 64, FAKE, 4, 64, 1e-6, 0, st) == DTYPE
    assert lib.ts_rmsnorm_fwd(FAKE, 64, 1, FAKE, 2, FAKE, 64, FAKE, 4, 64, 1e-6, 0, st) == DTYPE
    assert lib.ts_rmsnorm_fwd(NULL, 64, 1, FAKE, 1, FAKE, 64, FAKE, 4, 64, 1e-6, 0, st) == INVALID
    assert lib.ts_rmsnorm_fwd(FAKE, 32, 1, FAKE, 1, FAKE, 64, FAKE, 4, 64, 1e-6, 0, st) == SHAPE
    assert lib.ts_rmsnorm_fwd(FAKE, 64, 1, FAKE, 1, FAKE, 64, FAKE, 4, 64, -1.0, 0, st) == INVALID
    assert lib.ts_rmsnorm_fwd(FAKE, 64, 1, FAKE, 1, FAKE, 64, FAKE, 4, 64, 1e-6, 5, st) == INVALID
    assert b"round_mode" in lib.ts_last_error()
    # an empty batch is a no-op
    assert lib.ts_rmsnorm_fwd(NULL, 64, 1, NULL, 1, NULL, 64, NULL, 0, 64, 1e-6, 0, st) == TS_OK


def test_rmsnorm_bwd_validation(lib):
    st = NULL
    need = lib.ts_rmsnorm_bwd_workspace_size(16384, 4096)
    assert need > 0 and need % 4 == 0
    assert lib.ts_rmsnorm_bwd_workspace_size(0, 4096) == 0
    # dW requested with a too-small workspace
    rc = lib.ts_rmsnorm_bwd(FAKE, 4096, FAKE, 4096, 1, FAKE, 1, FAKE, FAKE, 4096, FAKE,
                            FAKE, need - 16, 16384, 4096, st)
    assert rc == WORKSPACE, _lib.last_error()
    # dW without a weight
    rc = lib.ts_rmsnorm_bwd(FAKE, 4096, FAKE, 4096, 1, NULL, 1, FAKE, FAKE, 4096, FAKE,
                            FAKE, need, 16384, 4096, st)
    assert rc == INVALID
    rc = lib.ts_rmsnorm_bwd(NULL, 4096, FAKE, 4096, 1, FAKE, 1, FAKE, FAKE, 4096, NULL,
                            NULL, 0, 16, 4096, st)
    assert rc == INVALID


def _rope(lib, **kw):
    a = dict(q_in=FAKE, q_out=FAKE, qs=(4096, 512, 128), qos=(4096, 512, 128), Hq=4,
             k_in=NULL, k_out=NULL, ks=(0, 0, 0), kos=(0, 0, 0), Hk=0, dtype=1, B=2, S=8, D=128,
             cos=FAKE, sin=FAKE, tab_dtype=0, tab_ld=64, rows=8, inv=NULL, pos_div=1.0,
             ascale=1.0, pos=NULL, psb=0, pss=0, off=0, il=0, bwd=0)
    a.update(kw)
    return lib.ts_rope_apply(a["q_in"], a["q_out"], *a["qs"], *a["qos"], a["Hq"], a["k_in"],
                             a["k_out"], *a["ks"], *a["kos"], a["Hk"], a["dtype"], a["B"], a["S"],
                             a["D"], a["cos"], a["sin"], a["tab_dtype"], a["tab_ld"], a["rows"],
                             a["inv"], a["pos_div"], a["ascale"], a["pos"], a["psb"], a["pss"],
                             a["off"],
                             a["il"], a["bwd"], NULL)


def test_rope_validation(lib):
    assert _rope(lib, cos=NULL, sin=NULL, inv=FAKE, ascale=0.0) == INVALID
    assert _rope(lib, cos=NULL, sin=NULL, inv=FAKE, ascale=float("inf")) == INVALID
    assert _rope(lib, D=127) == SHAPE
    assert _rope(lib, D=1024) == SHAPE
    assert _rope(lib, rows=7) == SHAPE  # positions 0..7 need 8 table rows
    assert b"exceed" in lib.ts_last_error()
    assert _rope(lib, off=1) == SHAPE
    assert _rope(lib, sin=NULL) == INVALID
    assert _rope(lib, cos=NULL, sin=NULL) == INVALID  # neither tables nor inv_freq
    assert _rope(lib, Hk=2) == INVALID  # K heads without K pointers
    assert _rope(lib, il=2) == INVALID
    assert _rope(lib, dtype=9) == DTYPE
    assert _rope(lib, S=0) == TS_OK
    # empty tensors carry NULL data pointers: no tokens, nothing to check or launch
    assert _rope(lib, S=0, q_in=NULL, q_out=NULL) == TS_OK
    assert _rope(lib, B=0, q_in=NULL, q_out=NULL, Hk=2) == TS_OK
    assert _rope(lib, q_in=NULL) == INVALID  # tokens but no Q data


def test_ce_validation(lib):
    st = NULL
    f = lambda **k: lib.ts_ce_fwd(k.get("x", FAKE), k.get("ld", 128), k.get("dt", 1),
                                  k.get("lab", FAKE), k.get("N", 4), k.get("V", 128), -100,
                                  k.get("scale", 0.0), k.get("cap", 0.0), k.get("ls", 0.0),
                                  FAKE, FAKE, st)
    assert f(ld=64) == SHAPE
    assert f(V=0) == SHAPE
    assert f(ls=1.0) == INVALID
    assert f(cap=-1.0) == INVALID
    assert f(lab=NULL) == INVALID
    assert f(dt=5) == DTYPE
    assert f(N=0) == TS_OK
    # in-place backward needs the logits layout
    rc = lib.ts_ce_bwd(FAKE, 128, 1, FAKE, FAKE, FAKE, 1, 1.0, FAKE, 256, 1, 4, 128, -100,
                       0.0, 0.0, 0.0, st)
    assert rc == INVALID
    rc = lib.ts_ce_bwd(FAKE, 128, 1, FAKE, FAKE, FAKE, 1, 1.0, FAKE, 128, 2, 4, 128, -100,
                       0.0, 0.0, 0.0, st)
    assert rc == DTYPE


def test_vocab_parallel_validation(lib):
    st = NULL
    stats = lambda **k: lib.ts_ce_vocab_shard_stats(
        k.get("x", FAKE), k.get("ld", 128), k.get("dt", 1), k.get("t", FAKE), k.get("N", 4),
        k.get("Vp", 128), k.get("v0", 0), k.get("out", FAKE), st)
    assert stats(ld=64) == SHAPE
    assert stats(Vp=0) == SHAPE
    assert stats(N=-1) == SHAPE
    assert stats(v0=-5) == INVALID
    assert stats(t=NULL) == INVALID
    assert stats(out=NULL) == INVALID
    assert stats(dt=7) == DTYPE
    assert stats(Vp=1 << 29, ld=1 << 29) == SHAPE
    assert stats(N=0, out=NULL) == TS_OK
    merge = lambda **k: lib.ts_ce_vocab_merge(
        k.get("s", FAKE), k.get("P", 2), k.get("self", 0), k.get("N", 4), k.get("Vp", 64),
        k.get("a", 0.0), k.get("lse", FAKE), k.get("loss", FAKE), st)
    assert merge(P=0) == INVALID
    assert merge(self=2) == INVALID
    assert merge(self=-1) == INVALID
    assert merge(Vp=0) == SHAPE
    assert merge(a=1.5) == INVALID
    assert merge(loss=NULL) == INVALID
    assert merge(N=0, s=NULL) == TS_OK
    bwd = lambda **k: lib.ts_ce_vocab_shard_bwd(
        k.get("x", FAKE), k.get("ld", 128), k.get("dt", 1), k.get("t", FAKE), FAKE,
        k.get("go", FAKE), 1.0, k.get("N", 4), k.get("Vp", 128), 0, k.get("a", 0.0),
        k.get("g", FAKE), k.get("ldg", 128), k.get("gdt", 1), st)
    assert bwd(gdt=2) == DTYPE  # fp16 grad for bf16 logits
    assert bwd(gdt=9) == DTYPE
    assert bwd(ldg=64) == SHAPE
    assert bwd(a=-0.1) == INVALID
    assert bwd(go=NULL) == INVALID
    assert bwd(g=NULL) == INVALID
    assert bwd(N=0, g=NULL) == TS_OK


def test_flce_vocab_validation(lib):
    st = NULL
    ws_need = lib.ts_flce_vocab_workspace_size(64, 256)
    assert ws_need > 64 * 256 * 2
    assert lib.ts_flce_vocab_workspace_size(0, 256) == 0
    fwd = lambda **k: lib.ts_flce_vocab_fwd(
        k.get("h", FAKE), k.get("ldh", 128), k.get("w", FAKE), k.get("ldw", 128), k.get("lab", FAKE),
        k.get("N", 64), k.get("H", 128), k.get("Vp", 256), k.get("v0", 0), k.get("stats", FAKE),
        k.get("ws", FAKE), k.get("wsb", ws_need), st)
    assert fwd(N=60) == SHAPE       # not a multiple of 8
    assert fwd(H=100) == SHAPE
    assert fwd(Vp=0) == SHAPE
    # any shard width: the shard's logits rows are padded to whole 16-byte vectors
    assert lib.ts_flce_vocab_workspace_size(64, 1001) >= 64 * 1008 * 2
    assert fwd(Vp=1001, wsb=0) == WORKSPACE  # past the shape checks, stopped before a launch
    assert fwd(ldh=64) == SHAPE
    assert fwd(Vp=1 << 23) == SHAPE
    assert fwd(v0=-8) == INVALID
    assert fwd(lab=NULL) == INVALID
    assert fwd(stats=NULL) == INVALID
    assert fwd(wsb=ws_need - 1) == WORKSPACE
    assert fwd(ws=NULL) == WORKSPACE
    bwd = lambda **k: lib.ts_flce_vocab_bwd(
        FAKE, 128, FAKE, 128, FAKE, 64, 128, 256, 0, k.get("sa", FAKE), k.get("P", 2), -100,
        k.get("red", 0), k.get("loss", FAKE), NULL, NULL, FAKE, FAKE, FAKE, k.get("wsb", ws_need), st)
    assert bwd(P=0) == INVALID
    assert bwd(sa=NULL) == INVALID
    assert bwd(red=3) == INVALID
    assert bwd(loss=NULL) == INVALID
    assert bwd(wsb=16) == WORKSPACE


def test_scale_and_rescale_validation(lib):
    st = NULL
    assert lib.ts_scale_inplace(FAKE, -1, 1, FAKE, st) == SHAPE
    assert lib.ts_scale_inplace(NULL, 12, 1, FAKE, st) == INVALID
    assert lib.ts_scale_inplace(FAKE, 16, 9, FAKE, st) == DTYPE
    assert lib.ts_scale_inplace(FAKE, 16, 1, NULL, st) == INVALID
    assert lib.ts_rescale_inplace(FAKE, 16, 1, FAKE, NULL, NULL, st) == INVALID
    hint = ctypes.c_void_p(0x2000)
    assert lib.ts_rescale_inplace(FAKE, 16, 1, hint, FAKE, hint, st) == INVALID
    assert b"aliases" in lib.ts_last_error()
    assert lib.ts_rescale_inplace(FAKE, 16, 9, FAKE, FAKE, NULL, st) == DTYPE
    assert lib.ts_scale_inplace(NULL, 0, 1, FAKE, st) == TS_OK


def test_add_rmsnorm_fwd_validation(lib):
    st = NULL
    args = lambda **kw: [kw.get("x", FAKE), kw.get("ldx", 64), kw.get("r", FAKE), kw.get("ldr", 64),
                         kw.get("dt", 1), FAKE, 1, FAKE, 64, kw.get("h", FAKE), kw.get("ldh", 64),
                         FAKE, kw.get("rows", 4), 64, 1e-6, kw.get("mode", 1), st]
    assert lib.ts_add_rmsnorm_fwd(*args(r=NULL)) == INVALID
    assert lib.ts_add_rmsnorm_fwd(*args(ldr=32)) == SHAPE
    assert lib.ts_add_rmsnorm_fwd(*args(ldh=32)) == SHAPE
    assert lib.ts_add_rmsnorm_fwd(*args(dt=5)) == DTYPE
    assert lib.ts_add_rmsnorm_fwd(*args(mode=3)) == INVALID
    # h_out may be NULL (its stride is then ignored); an empty batch is a no-op
    assert lib.ts_add_rmsnorm_fwd(*args(h=NULL, ldh=0, rows=0)) == TS_OK


def test_swiglu_validation(lib):
    st = NULL
    assert lib.ts_swiglu_fwd(FAKE, FAKE, FAKE, -1, 1, st) == SHAPE
    assert lib.ts_swiglu_fwd(FAKE, FAKE, FAKE, 16, 7, st) == DTYPE
    assert lib.ts_swiglu_fwd(FAKE, NULL, FAKE, 16, 1, st) == INVALID
    assert lib.ts_swiglu_bwd(FAKE, FAKE, FAKE, FAKE, NULL, 16, 1, st) == INVALID
    assert lib.ts_swiglu_fwd(NULL, NULL, NULL, 0, 1, st) == TS_OK
    assert lib.ts_swiglu_bwd(NULL, NULL, NULL, NULL, NULL, 0, 1, st) == TS_OK


def test_flce_validation(lib):
    st = NULL
    N, H, V = 64, 64, 128
    ws = lib.ts_flce_workspace_size(N, H, V, 0, 1)
    assert ws > 0 and lib.ts_flce_workspace_size(0, H, V, 0, 1) == 0

    def call(ldh=H, ldw=H, n=N, h=H, v=V, reduction=0, loss=FAKE, wsb=ws, hidden=FAKE, flags=0):
        return lib.ts_flce_fwd_bwd(hidden, ldh, FAKE, ldw, FAKE, n, h, v, -100, reduction, loss,
                                   NULL, NULL, FAKE, FAKE, 0, flags, FAKE, wsb, st)

    assert call(h=60, ldh=64, ldw=64) == SHAPE          # H not a multiple of 8
    assert call(ldh=32) == SHAPE                        # row stride below H
    assert call(ldh=72 + 4) == SHAPE                    # row stride not a multiple of 8
    assert call(ldh=(1 << 22) + 8) == SHAPE             # offsets would leave 32 bits
    assert b"row strides" in lib.ts_last_error()
    assert call(ldw=(1 << 22) + 8) == SHAPE
    assert call(v=(1 << 22) + 8) == SHAPE
    assert call(reduction=2) == INVALID
    assert call(loss=NULL) == INVALID
    assert call(hidden=NULL) == INVALID
    assert call(wsb=ws - 256) == WORKSPACE
    assert call(flags=4) == INVALID
    # the flags given to ts_flce_workspace_size are accepted (TS_FLCE_GRADS is ignored
    # here): these calls pass the flag check and stop at the missing workspace
    for flags in (1, 2, 3):
        assert call(flags=flags, wsb=0) == WORKSPACE, flags
    assert call(flags=5, wsb=0) == INVALID
    # bf16 accumulation needs no V x H fp32 sum: smaller than fp32 accumulation over chunks
    assert lib.ts_flce_workspace_size(1024, 256, 4096, 256, 3) + 4096 * 256 * 4 == \
        lib.ts_flce_workspace_size(1024, 256, 4096, 256, 1)


def test_flce_two_pass_validation(lib):
    st = NULL
    N, H, V = 65, 64, 128  # any token count
    wf = lib.ts_flce_forward_workspace_size(N, V)
    wb = lib.ts_flce_backward_workspace_size(N, H, V, 0)
    assert wf > 0 and wb > 0 and lib.ts_flce_forward_workspace_size(0, V) == 0
    # more vocabulary chunks: a smaller dlogits buffer plus the fp32 grad_hidden sum
    assert lib.ts_flce_backward_workspace_size(N, H, 4096, 256) < \
        lib.ts_flce_backward_workspace_size(N, H, 4096, 4096) + N * H * 4

    def fwd(n=N, h=H, v=V, ldh=H, red=0, cap=0.0, sc=0.0, temp=1.0, loss=FAKE, wsb=wf,
            hidden=FAKE):
        return lib.ts_flce_forward(hidden, ldh, FAKE, H, FAKE, n, h, v, -100, red, cap, sc, temp,
                                   loss, NULL, NULL, FAKE, wsb, st)

    assert fwd(h=60, ldh=64) == SHAPE
    # any V passes the shape checks (rows of the library's logits are padded): these calls
    # stop at the missing workspace, before anything is launched
    assert fwd(v=100, wsb=0) == WORKSPACE
    assert fwd(v=50257, wsb=0) == WORKSPACE
    assert fwd(ldh=32) == SHAPE
    assert fwd(red=3) == INVALID
    assert fwd(loss=NULL) == INVALID      # mean needs the scalar
    assert fwd(cap=-1.0) == INVALID
    assert fwd(temp=0.0) == INVALID
    assert fwd(sc=float("nan")) == INVALID
    assert fwd(hidden=NULL) == INVALID
    assert fwd(wsb=wf - 256) == WORKSPACE
    assert fwd(n=0, loss=NULL, red=2) == TS_OK  # nothing to do

    def bwd(dl_stride=0, lse=FAKE, dloss=FAKE, wsb=wb, gh=FAKE, gw=FAKE, temp=1.0):
        return lib.ts_flce_backward(FAKE, H, FAKE, H, FAKE, N, H, V, -100, 2, 0.0, 0.0, temp, lse,
                                    dloss, dl_stride, gh, gw, 0, FAKE, wsb, st)

    assert bwd(dl_stride=-1) == INVALID
    assert bwd(lse=NULL) == INVALID
    assert bwd(dloss=NULL) == INVALID
    assert bwd(temp=-1.0) == INVALID
    assert bwd(gh=ctypes.c_void_p(0x1008)) == INVALID   # unaligned
    assert bwd(wsb=wb - 256) == WORKSPACE
    assert bwd(gh=NULL, gw=NULL) == TS_OK   # no gradient requested: nothing launched

    # the stored-logits pair: the forward's checks plus the logits buffer
    def fwd_keep(logits=FAKE, red=0, temp=1.0, wsb=wf, n=N):
        return lib.ts_flce_forward_keep(FAKE, H, FAKE, H, FAKE, n, H, V, -100, red, 0.0, 0.0,
                                        temp, FAKE, NULL, NULL, logits, FAKE, wsb, st)

    assert fwd_keep(logits=NULL) == INVALID
    assert fwd_keep(logits=ctypes.c_void_p(0x1008)) == INVALID  # unaligned
    assert fwd_keep(red=3) == INVALID
    assert fwd_keep(temp=0.0) == INVALID
    assert fwd_keep(wsb=wf - 256) == WORKSPACE
    wk = lib.ts_flce_backward_kept_workspace_size(N)
    assert wk >= N * 4 and lib.ts_flce_backward_kept_workspace_size(0) == 0

    def bwd_kept(logits=FAKE, lse=FAKE, dloss=FAKE, dl_stride=0, wsb=wk, gh=FAKE, gw=FAKE):
        return lib.ts_flce_backward_kept(FAKE, H, FAKE, H, FAKE, N, H, V, -100, 2, 0.0, 0.0,
                                         1.0, lse, dloss, dl_stride, logits, gh, gw, FAKE, wsb,
                                         st)

    assert bwd_kept(logits=NULL) == INVALID
    assert bwd_kept(logits=ctypes.c_void_p(0x1008)) == INVALID
    assert bwd_kept(lse=NULL) == INVALID
    assert bwd_kept(dloss=NULL) == INVALID
    assert bwd_kept(dl_stride=-1) == INVALID
    assert bwd_kept(gw=ctypes.c_void_p(0x1008)) == INVALID
    assert bwd_kept(wsb=wk - 256) == WORKSPACE
    assert bwd_kept(gh=NULL, gw=NULL) == TS_OK


def test_noalloc_rejects_shapes_beyond_the_scratch(lib):
    """ts_rmsnorm_bwd_noalloc refuses partials above its 16 MiB device scratch before any
    HIP call (so these made-up pointers are never used)."""
    cap = int(lib.ts_rmsnorm_bwd_noalloc_max_bytes())
    assert cap == 16 << 20
    rows, cols = 65536, 65536  # the generic path's partials: rows / 64 x cols x 4 bytes
    assert int(lib.ts_rmsnorm_bwd_workspace_size(rows, cols)) > cap
    status = lib.ts_rmsnorm_bwd_noalloc(FAKE, cols, FAKE, cols, _lib.TS_BF16, FAKE, _lib.TS_BF16,
                                        FAKE, FAKE, cols, FAKE, rows, cols, NULL)
    assert status == WORKSPACE
    assert b"device scratch" in lib.ts_last_error()
