"""C-ABI checks that need no GPU: the library loads, exports every function
``include/linatt_hip.h`` declares, and rejects bad arguments with the
documented status codes before touching the device."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "linatt_hip.h")


@pytest.fixture(scope="module")
def lib():
    from linatt_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from linatt_amd import build
        build.build()
    return _lib.load()


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(linatt_[a-z0-9_]+)\s*\(", text)))


def test_exports_every_declared_symbol(lib):
    names = declared_functions()
    assert len(names) >= 6
    for n in names:
        assert hasattr(lib, n), f"{n} declared in linatt_hip.h but not exported"


def test_python_signatures_cover_header():
    from linatt_amd import _lib
    assert set(declared_functions()) == set(_lib.SIGNATURES)


def declared_prototypes():
    """{name: [parameter declarations]} from the header's prototypes."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for m in re.finditer(r"\b(linatt_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        params = [p.strip() for p in m.group(2).split(",") if p.strip()]
        out[m.group(1)] = [] if params == ["void"] else params
    return out


def test_python_signatures_match_prototypes():
    """Each ctypes signature has the header prototype's arity, and pointer,
    float, int and size_t parameters line up."""
    from linatt_amd import _lib
    protos = declared_prototypes()
    assert set(protos) == set(_lib.SIGNATURES)
    for name, params in protos.items():
        res, args = _lib.SIGNATURES[name]
        assert len(args) == len(params), (name, len(args), len(params))
        for decl, ct in zip(params, args):
            if "*" in decl:
                assert ct is ctypes.c_void_p, (name, decl)
            elif decl.startswith("float"):
                assert ct is ctypes.c_float, (name, decl)
            elif decl.startswith("size_t"):
                assert ct is ctypes.c_size_t, (name, decl)
            else:
                assert ct is ctypes.c_int, (name, decl)


def test_version_and_support(lib):
    assert lib.linatt_abi_version() == 3
    BF16, F32, F16 = 1, 0, 2
    for dt in (BF16, F32, F16):
        for M in (1, 2, 4):
            assert lib.linatt_kata_supported(dt, 64, 64, M, 0, 0) == 1
            assert lib.linatt_kata_supported(dt, 64, 64, M, 1, 0) == 1
            assert lib.linatt_kata_supported(dt, 64, 64, M, 0, 1) == 1
            assert lib.linatt_kata_supported(dt, 64, 64, M, 1, 1) == 0  # decay is concat-only
    assert lib.linatt_kata_supported(BF16, 48, 64, 3, 0, 0) == 0
    # the offset-gated mixer's shape (groups of 32 padded to 64): concat, sum, decay
    for dt in (BF16, F32, F16):
        assert lib.linatt_kata_supported(dt, 128, 64, 2, 0, 1) == 1
        assert lib.linatt_kata_supported(dt, 128, 64, 2, 1, 0) == 1
    # -<o,dO> and scale^2/den rows (256-byte rounded); bf16 adds the prescaled dO
    assert lib.linatt_kata_bwd_workspace_bytes(2, 10, 3, 64, F32) == 512  # 480 rounded up
    assert lib.linatt_kata_bwd_workspace_bytes(2, 10, 3, 64, F16) == 512
    assert lib.linatt_kata_bwd_workspace_bytes(2, 10, 3, 64, BF16) == 512 + 2 * 10 * 3 * 64 * 2
    assert lib.linatt_kata_bwd_workspace_bytes(0, 10, 3, 64, BF16) == 0


def test_gen_state_rows_full_and_packed(lib):
    from linatt_amd.kata_cache import state_rows
    PK = 4  # LINATT_KATA_PACKED_STATE
    for dk, M in ((64, 1), (64, 2), (64, 4), (128, 2), (128, 8)):
        E = dk // M
        for var, name, G in ((0, "concat", M), (1, "sum", 1)):
            assert lib.linatt_kata_gen_state_rows(dk, M, var) == G * E * E == state_rows(dk, M, name)
            assert lib.linatt_kata_gen_state_rows(dk, M, var | PK) == G * E * (E + 1) // 2 \
                == state_rows(dk, M, name, True)
    assert lib.linatt_kata_gen_state_rows(64, 3, 0) == 0
    assert lib.linatt_kata_gen_state_rows(64, 2, 2) == 0  # no variant 2
    assert lib.linatt_kata_gen_state_rows(64, 2, 2 | PK) == 0


def test_gen_state_rejects_unknown_variant_bits(lib):
    null = None
    for var in (2, 2 | 4, 8):
        assert lib.linatt_kata_gen_decode(FAKE, FAKE, FAKE, null, FAKE, FAKE, FAKE, 1, 2, 64, 64, 2,
                                          var, 0.25, 1e-6, 1, null) == -1
        assert b"unknown KATA variant" in lib.linatt_last_error()


def test_gen_state_alignment_checked_before_launch(lib):
    odd = ctypes.c_void_p((1 << 20) + 2)  # 2-byte aligned only, never dereferenced
    null = None
    assert lib.linatt_kata_gen_readout(odd, null, FAKE, FAKE, FAKE, FAKE, 1, 8, 2, 64, 64, 2, 0,
                                       0.25, 1e-6, 1, null) == -1
    assert b"16-byte aligned" in lib.linatt_last_error()
    assert lib.linatt_kata_gen_update(odd, FAKE, null, FAKE, FAKE, 0, 1, 8, 2, 64, 64, 2, 0, 0.25, 1,
                                      null) == -1
    assert b"16-byte aligned" in lib.linatt_last_error()
    assert lib.linatt_kata_gen_update(FAKE, odd, null, FAKE, FAKE, 0, 1, 8, 2, 64, 64, 2, 0, 0.25, 1,
                                      null) == -1


FAKE = ctypes.c_void_p(1 << 20)  # aligned, never dereferenced on the host


def _fwd(lib, **kw):
    a = dict(q=FAKE, k=FAKE, v=FAKE, c=None, o=FAKE, den=FAKE, B=1, T=8, HQ=2, H=2, dk=64,
             dv=64, M=4, scale=0.25, variant=0, dtype=1, stream=None)
    a.update(kw)
    return lib.linatt_kata_fwd(a["q"], a["k"], a["v"], a["c"], a["o"], a["den"], a["B"], a["T"],
                               a["HQ"], a["H"], a["dk"], a["dv"], a["M"], a["scale"],
                               a["variant"], a["dtype"], a["stream"])


def test_fwd_argument_errors(lib):
    EINVAL, EUNSUP = -1, -2
    assert _fwd(lib, T=0) == EINVAL
    assert b"non-positive" in lib.linatt_last_error()
    assert _fwd(lib, HQ=3, H=2) == EINVAL
    assert b"GQA" in lib.linatt_last_error()
    assert _fwd(lib, dk=64, M=3) == EINVAL
    assert _fwd(lib, scale=0.0) == EINVAL
    assert _fwd(lib, variant=7) == EINVAL
    assert _fwd(lib, dtype=9) == EINVAL
    assert _fwd(lib, q=None) == EINVAL
    assert _fwd(lib, k=ctypes.c_void_p((1 << 20) + 2)) == EINVAL
    assert b"aligned" in lib.linatt_last_error()
    assert _fwd(lib, c=FAKE, variant=1) == EUNSUP
    assert _fwd(lib, dk=48, M=3) == EUNSUP
    assert b"no kernel compiled" in lib.linatt_last_error()


def test_bwd_argument_errors(lib):
    EINVAL, EUNSUP = -1, -2
    f = lambda **kw: lib.linatt_kata_bwd(  # noqa: E731
        FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, kw.get("ws", FAKE),
        1, 8, 2, 2, kw.get("dk", 64), 64, kw.get("M", 4), 0.25, 0, 1, None)
    assert f(ws=None) == EINVAL
    assert f(dk=48, M=3) == EUNSUP
    assert f(dk=64, M=5) == EINVAL


def test_python_layer_rejects_cpu_tensors(lib):
    import torch
    from linatt_amd import parallel_kata_attn as P
    q = torch.randn(1, 4, 1, 64)
    with pytest.raises(RuntimeError, match="only on a ROCm GPU"):
        P.parallel_kata_attn_fwd(q, q, q)


def test_noalloc_rejects_oversized_before_device_work(lib):
    EINVAL = -1
    assert lib.linatt_noalloc_scratch_bytes() == 32 << 20
    # bf16 B8 T4096 HQ12 dv64 needs ~51 MiB of workspace: refused with a clear
    # message before any HIP call (null pointers would also be refused later)
    st = lib.linatt_kata_bwd_noalloc(None, None, None, None, None, None, None, None, None,
                                     8, 4096, 12, 12, 64, 64, 4, 0.25, 0, 1, None)
    assert st == EINVAL
    assert b"exceeds the fixed scratch" in lib.linatt_last_error()
    st = lib.linatt_kata_bwd_noalloc(None, None, None, None, None, None, None, None, None,
                                     0, 8, 2, 2, 64, 64, 4, 0.25, 0, 1, None)
    assert st == EINVAL


def _qk(lib, bwd=False, **kw):
    a = dict(x=FAKE, w=FAKE, b=None, cache=None, nw=None, y=FAKE, B=1, T=8, H=2, D=64, W=4,
             act=1, norm=1, eps=1e-5, rw=64, rot=64, base=10000.0, offset=0, inter=1, dtype=1)
    a.update(kw)
    if bwd:
        return lib.linatt_qk_prologue_bwd(
            a["x"], a["w"], a["b"], a["cache"], a["nw"], FAKE, FAKE, FAKE, None,
            kw.get("dnw"), kw.get("ws", FAKE), a["B"], a["T"], a["H"], a["D"], a["W"], a["act"],
            a["norm"], a["eps"], a["rw"], a["rot"], a["base"], a["offset"], a["inter"],
            a["dtype"], None)
    return lib.linatt_qk_prologue_fwd(
        a["x"], a["w"], a["b"], a["cache"], a["nw"], a["y"], kw.get("co"), a["B"], a["T"], a["H"],
        a["D"], a["W"], a["act"], a["norm"], a["eps"], a["rw"], a["rot"], a["base"],
        a["offset"], a["inter"], a["dtype"], None)


def test_qk_prologue_argument_errors(lib):
    EINVAL, EUNSUP = -1, -2
    assert _qk(lib, T=0) == EINVAL
    assert _qk(lib, D=48, rw=48, rot=48) == EUNSUP
    assert b"head dim" in lib.linatt_last_error()
    assert _qk(lib, W=5) == EUNSUP
    assert _qk(lib, norm=3) == EINVAL
    assert _qk(lib, norm=2, nw=FAKE) == EINVAL
    assert b"L2 norm takes no weight" in lib.linatt_last_error()
    assert _qk(lib, rw=24, rot=24) == EINVAL          # 24 does not divide 64
    assert _qk(lib, rw=16, rot=18) == EINVAL          # rot_dim > rope_width
    assert _qk(lib, rw=16, rot=12, inter=0) == EUNSUP  # half-split needs rot_dim % 8 == 0
    assert _qk(lib, offset=-1) == EINVAL
    assert _qk(lib, base=1.0) == EINVAL
    assert _qk(lib, x=ctypes.c_void_p((1 << 20) + 2)) == EINVAL
    assert _qk(lib, dtype=9) == EINVAL
    assert _qk(lib, bwd=True, ws=None) == EINVAL
    assert _qk(lib, bwd=True, dnw=FAKE) == EINVAL     # dnorm_weight without norm_weight
    # rot_dim 0 switches the rotation off and ignores rope_width
    assert _qk(lib, rot=0, rw=-3, T=0) == EINVAL
    assert b"non-positive" in lib.linatt_last_error()
    # an in-place cache update races across 16-token runs
    c0, c1 = ctypes.c_void_p(1 << 24), ctypes.c_void_p((1 << 24) + 64)
    assert _qk(lib, T=17, cache=c0, co=c1) == EINVAL
    assert b"cache_out overlaps cache_in" in lib.linatt_last_error()


def test_short_conv_cache_alias_rejected(lib):
    EINVAL = -1
    c0, c1 = ctypes.c_void_p(1 << 24), ctypes.c_void_p((1 << 24) + 2 * 8 * 4 - 2)
    st = lib.linatt_short_conv_fwd(FAKE, FAKE, None, c0, FAKE, c1, 1, 40, 8, 4, 1, 1, None)
    assert st == EINVAL and b"cache_out overlaps cache_in" in lib.linatt_last_error()
    st = lib.linatt_short_conv_fwd(FAKE, FAKE, None, c0, FAKE, c0, 2, 17, 8, 4, 1, 0, None)
    assert st == EINVAL


def test_qk_prologue_workspace_bytes(lib):
    # convolution partials [B ntb][C][W + 1] + norm-weight partials [B ntb][H / h][D], h the
    # heads per block (the largest divisor of H with h D / 4 <= 256 lanes)
    B, T, H, D, W = 2, 33, 3, 64, 4
    np_, C = B * 3, H * D
    assert lib.linatt_qk_prologue_bwd_workspace_bytes(B, T, H, D, W) == \
        (np_ * C * (W + 1) + np_ * 1 * D) * 4
    B, T = 8, 2048  # 12 heads of 64 in one block of 192 lanes
    np_ = B * 128
    assert lib.linatt_qk_prologue_bwd_workspace_bytes(B, T, 12, 64, W) == \
        (np_ * 768 * (W + 1) + np_ * 1 * 64) * 4
    # 20 heads of 128: 32 lanes each, h = 5 (8 would not divide 20) -> 4 blocks per row
    assert lib.linatt_qk_prologue_bwd_workspace_bytes(1, 16, 20, 128, W) == \
        (1 * 2560 * (W + 1) + 1 * 4 * 128) * 4
    assert lib.linatt_qk_prologue_bwd_workspace_bytes(B, T, H, D, 5) == 0


def test_qk_prologue_python_checks():
    import torch
    from linatt_amd import mixer
    x = torch.randn(1, 4, 128)
    w = torch.randn(128, 1, 4)
    with pytest.raises(ValueError, match="multiple of head_dim"):
        mixer.qk_prologue(x, w, head_dim=48)
    with pytest.raises(ValueError, match="norm_weight is only used"):
        mixer.qk_prologue(x, w, head_dim=64, norm="l2", norm_weight=torch.ones(64))
    with pytest.raises(ValueError, match="norm must be"):
        mixer.qk_prologue(x, w, head_dim=64, norm="layer")
    with pytest.raises(RuntimeError, match="only on a ROCm GPU"):
        mixer.qk_prologue(x, w, head_dim=64)
