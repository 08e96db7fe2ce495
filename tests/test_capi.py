"""C-ABI checks that need no GPU: the library loads, exports every symbol the
header declares, and its host-side validation rejects bad arguments with a
negative status and a message (no kernel is launched on these paths)."""

import ctypes
import os
import re

import pytest

from redpanda_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                      "include", "redpanda_hip.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rp_[a-z_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return _lib.open_library()


def test_header_and_binding_agree():
    assert _declared() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol(lib):
    for name in _declared():
        assert hasattr(lib, name), name


def test_abi_version(lib):
    assert lib.rp_abi_version() == _lib.ABI_VERSION


def _good_args(**kw):
    a = _lib.ScanArgs()
    a.B, a.L, a.D, a.N, a.NR, a.NT = 2, 64, 128, 40, 32, 8
    a.dtype_delta = a.dtype_u = a.dtype_B = a.dtype_C = _lib.RP_BF16
    fake = 0x10000  # never dereferenced: validation only
    a.delta = a.u = a.Bc = a.Cc = fake
    a.delta_sb, a.delta_sl = 64 * 128, 128
    a.u_sb, a.u_sl = 64 * 128, 128
    a.Bc_sb, a.Bc_sl = 64 * 40, 40
    a.Cc_sb, a.Cc_sl = 64 * 40, 40
    a.A_real = a.A_imag = a.track = fake
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def test_valid_args_pass_check(lib):
    assert lib.rp_scan_check(ctypes.byref(_good_args())) == 0


@pytest.mark.parametrize("field,value,needle", [
    ("N", 41, "NR+NT"),
    ("NR", -1, "negative"),
    ("N", 0, "outside"),
    ("dtype_u", 7, "dtype"),
    ("bidirectional", 2, "bidirectional"),
    ("delta", None, "NULL"),
    ("track", None, "track"),
    ("u_sl", -5, "stride"),
    ("delta_softplus", 2, "delta_softplus"),
    ("grad_in_storage", 2, "grad_in_storage"),
])
def test_invalid_scan_args_rejected(lib, field, value, needle):
    kw = {field: value}
    if field == "N" and value == 0:
        kw.update(NR=0, NT=0)
    a = _good_args(**kw)
    st = lib.rp_scan_check(ctypes.byref(a))
    assert st < 0
    assert needle in lib.rp_last_error().decode()


def test_state_too_large_is_unsupported(lib):
    a = _good_args(N=200, NR=192, NT=8)
    assert lib.rp_scan_check(ctypes.byref(a)) == -2


def test_workspace_queries(lib):
    a = _good_args()
    ck = lib.rp_scan_ckpt_bytes(ctypes.byref(a))
    wk = lib.rp_scan_bwd_work_bytes(ctypes.byref(a))
    assert ck > 0 and wk > 0 and wk % 256 == 0
    a1 = _good_args(L=1)  # a single step needs no stored checkpoint
    assert lib.rp_scan_ckpt_bytes(ctypes.byref(a1)) == 0
    sizes = [lib.rp_scan_ckpt_bytes(ctypes.byref(_good_args(L=L))) for L in (16, 64, 256)]
    assert sizes[0] < sizes[1] < sizes[2]  # one record per chunk boundary
    bad = _good_args(N=3)
    assert lib.rp_scan_ckpt_bytes(ctypes.byref(bad)) == -1


def test_final_state_rejected_for_bidirectional(lib):
    a = _good_args(bidirectional=1)
    out = _lib.ScanFwdOut(0x10000, None, 0x10000, 0x10000)
    assert lib.rp_scan_fwd(ctypes.byref(a), ctypes.byref(out), None) < 0
    assert "causal" in lib.rp_last_error().decode()


def test_bwd_workspace_too_small_rejected(lib):
    a = _good_args()
    f = 0x10000
    io = _lib.ScanBwdIO(dy=f, ckpt=f, d_delta=f, d_u=f, d_Bc=f, d_Cc=f, d_A_real=f,
                        d_A_imag=f, d_track=f, work=f, work_bytes=16)
    assert lib.rp_scan_bwd(ctypes.byref(a), ctypes.byref(io), None) == -4


def test_grad_in_storage_workspace(lib):
    # 16-bit gradients of a bidirectional scan: the first direction's fp32
    # (d_delta, d_u) sums join the workspace; causal scans write directly
    base = lib.rp_scan_bwd_work_bytes(ctypes.byref(_good_args(bidirectional=1)))
    wide = lib.rp_scan_bwd_work_bytes(ctypes.byref(_good_args(bidirectional=1, grad_in_storage=1)))
    assert wide - base == 2 * (2 * 64 * 128) * 4
    assert (lib.rp_scan_bwd_work_bytes(ctypes.byref(_good_args(grad_in_storage=1))) ==
            lib.rp_scan_bwd_work_bytes(ctypes.byref(_good_args())))
    f32 = dict(bidirectional=1, grad_in_storage=1, dtype_delta=_lib.RP_F32, dtype_u=_lib.RP_F32)
    assert (lib.rp_scan_bwd_work_bytes(ctypes.byref(_good_args(**f32))) ==
            lib.rp_scan_bwd_work_bytes(ctypes.byref(_good_args(bidirectional=1, dtype_delta=_lib.RP_F32,
                                                               dtype_u=_lib.RP_F32))))


def test_softplus_argument_checks(lib):
    # rejected before any launch; n = 0 launches nothing
    assert lib.rp_softplus(None, None, -1, None) < 0
    assert "n < 0" in lib.rp_last_error().decode()
    assert lib.rp_softplus(None, 0x10000, 8, None) < 0
    assert lib.rp_softplus(0x10002, 0x10000, 8, None) < 0
    assert "misaligned" in lib.rp_last_error().decode()
    assert lib.rp_softplus(None, None, 0, None) == 0


def _step_args(**kw):
    a = _lib.StepArgs()
    a.R, a.D, a.N, a.NR, a.NT = 16, 64, 20, 16, 4
    f = 0x10000
    a.delta = a.u = a.Bc = a.Cc = a.A_real = a.A_imag = a.track = a.Dskip = f
    a.h_in = a.beta_in = a.h_out = a.beta_out = a.y = f
    a.delta_sr = a.u_sr = 64
    a.Bc_sr = a.Cc_sr = 20
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def test_step_check(lib):
    assert lib.rp_step_check(ctypes.byref(_step_args())) == 0
    assert lib.rp_step_check(ctypes.byref(_step_args(beta_in=None))) < 0
    assert "together" in lib.rp_last_error().decode()
    assert lib.rp_step_check(ctypes.byref(_step_args(Bc_sr=3))) < 0
    assert lib.rp_step_check(ctypes.byref(_step_args(NT=5))) < 0


def test_step_broadcast_state_rules(lib):
    # one shared (D, N) input state read by every rollout, outputs elsewhere
    ok = dict(broadcast_state=1, h_in=0x100000, beta_in=0x200000, h_out=0x300000,
              beta_out=0x400000)
    assert lib.rp_step_check(ctypes.byref(_step_args(**ok))) == 0
    assert lib.rp_step_check(ctypes.byref(_step_args(**{**ok, "broadcast_state": 2}))) < 0
    assert lib.rp_step_check(ctypes.byref(_step_args(**{**ok, "delta_softplus": 2}))) < 0
    assert lib.rp_step_check(ctypes.byref(_step_args(**{**ok, "delta_softplus": 1}))) == 0
    assert lib.rp_step_check(ctypes.byref(_step_args(**{**ok, "h_in": None,
                                                         "beta_in": None}))) < 0
    # in place would let one rollout overwrite the state the others still read
    assert lib.rp_step_check(ctypes.byref(_step_args(**{**ok, "h_out": 0x100000}))) < 0
    assert "overlaps" in lib.rp_last_error().decode()
    # the output block (R*D*N*4 bytes) reaching into the shared input
    assert lib.rp_step_check(ctypes.byref(_step_args(**{**ok, "beta_out": 0x200000 - 64}))) < 0


def test_step_rank1_rules(lib):
    """Rank-1 beta rows (R, D + N): flags validated; beta_out may not overlap
    beta_in, since every channel tile of a rollout reads its B_prev part."""
    R, D, N = 16, 64, 20
    ok = dict(beta_rank1=1, h_in=0x100000, beta_in=0x200000, h_out=0x300000,
              beta_out=0x400000)
    assert lib.rp_step_check(ctypes.byref(_step_args(**ok))) == 0
    assert lib.rp_step_check(ctypes.byref(_step_args(**{**ok, "beta_rank1": 2}))) < 0
    assert lib.rp_step_check(ctypes.byref(_step_args(**{**ok, "reserved": 1}))) < 0
    assert lib.rp_step_check(ctypes.byref(_step_args(**{**ok, "beta_out": 0x200000}))) < 0
    assert "rank-1" in lib.rp_last_error().decode()
    # the input rows end at beta_in + R (D + N) 4 bytes
    end = 0x200000 + R * (D + N) * 4
    assert lib.rp_step_check(ctypes.byref(_step_args(**{**ok, "beta_out": end}))) == 0
    assert lib.rp_step_check(ctypes.byref(_step_args(**{**ok, "beta_out": end - 4}))) < 0
    # broadcast: one shared (D + N) row
    bc = dict(ok, broadcast_state=1)
    assert lib.rp_step_check(ctypes.byref(_step_args(**{**bc, "beta_out": 0x200000 + (D + N) * 4}))) == 0


def test_step_gate_rules(lib):
    ok = dict(z=0x500000, z_sr=2 * 64, dtype_z=_lib.RP_BF16)
    assert lib.rp_step_check(ctypes.byref(_step_args(**ok))) == 0
    assert lib.rp_step_check(ctypes.byref(_step_args(**{**ok, "dtype_z": 9}))) < 0
    assert lib.rp_step_check(ctypes.byref(_step_args(**{**ok, "z_sr": 63}))) < 0
    assert lib.rp_step_check(ctypes.byref(_step_args(**{**ok, "z": 0x500001}))) < 0
    assert lib.rp_step_check(ctypes.byref(_step_args(reserved2=1))) < 0


def test_initial_state_rules(lib):
    f = 0x10000
    assert lib.rp_scan_check(ctypes.byref(_good_args(h0=f, beta0=f))) == 0
    assert lib.rp_scan_check(ctypes.byref(_good_args(h0=f))) < 0
    assert "together" in lib.rp_last_error().decode()
    assert lib.rp_scan_check(ctypes.byref(_good_args(h0=f, beta0=f, bidirectional=1))) < 0
    assert "causal" in lib.rp_last_error().decode()
    assert lib.rp_scan_check(ctypes.byref(_good_args(h0=f, beta0=f, L=0))) < 0


def _header_struct_fields(name):
    """Field names of `typedef struct name {...} name;` in declaration order."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    body = re.search(r"typedef struct %s \{(.*?)\} %s;" % (name, name), text, flags=re.S).group(1)
    fields = []
    for decl in body.split(";"):
        decl = decl.strip()
        if not decl:
            continue
        # "int64_t B, L, D" / "const void* delta" / "float* y"
        head, *rest = [p.strip() for p in decl.split(",")]
        fields.append(re.findall(r"[A-Za-z_][A-Za-z0-9_]*", head)[-1])
        fields.extend(rest)
    return fields


@pytest.mark.parametrize("cname,pyname", [("rp_scan_args", "ScanArgs"),
                                          ("rp_scan_fwd_out", "ScanFwdOut"),
                                          ("rp_scan_bwd_io", "ScanBwdIO"),
                                          ("rp_step_args", "StepArgs"),
                                          ("rp_mixer_out_args", "MixerOutArgs"),
                                          ("rp_mixer_out_grad", "MixerOutGrad"),
                                          ("rp_bcnorm_args", "BcNormArgs"),
                                          ("rp_bcnorm_grad", "BcNormGrad"),
                                          ("rp_rmsnorm_args", "RmsNormArgs"),
                                          ("rp_ply_topk_args", "PlyTopkArgs"),
                                          ("rp_ply_gather_args", "PlyGatherArgs")])
def test_ctypes_structs_mirror_header(cname, pyname):
    py = [f[0] for f in getattr(_lib, pyname)._fields_]
    assert py == _header_struct_fields(cname)


def test_triton_scan_module_names():
    """The names the reference's callers import from `triton_scan`
    (engine/mamba.py:344, engine/train.py:711) exist with the same call shape."""
    import inspect

    from redpanda_amd import triton_scan

    for name in ("HAS_TRITON", "triton_trapezoidal_scan", "verify"):
        assert hasattr(triton_scan, name)
    params = list(inspect.signature(triton_scan.triton_trapezoidal_scan).parameters)
    assert params[:9] == ["delta", "u", "B_contracted", "C_contracted", "A_real", "A_imag",
                          "track", "n_rot", "n_state"]
    assert list(inspect.signature(triton_scan.verify).parameters) == ["device", "thorough", "verbose"]


def _mixer_args(**kw):
    a = _lib.MixerOutArgs()
    a.B, a.L, a.D, a.k_skip = 4, 64, 320, 2
    a.dtype_u, a.dtype_z = _lib.RP_BF16, _lib.RP_BF16
    n = 4 * 64 * 320
    a.y, a.out = 0x1000000, 0x2000000
    a.u, a.u_sb, a.u_sl = 0x3000000, 64 * 320, 320
    # z: the second half of an in_proj output of width 640
    a.z, a.z_sb, a.z_sl = 0x4000000 + 320 * 2, 64 * 640, 640
    a.Dskip = 0x5000000
    assert n * 4 < 0x1000000
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def test_mixer_out_check(lib):
    chk = lambda **kw: lib.rp_mixer_out_check(ctypes.byref(_mixer_args(**kw)))
    assert chk() == 0
    assert chk(out=0x1000000) == 0  # in place over y
    assert chk(k_skip=3) < 0 and "k_skip" in lib.rp_last_error().decode()
    assert chk(dtype_z=7) < 0
    assert chk(dtype_out=7) < 0
    assert chk(dtype_out=_lib.RP_BF16) == 0
    assert chk(dtype_out=_lib.RP_BF16, out=0x1000000) < 0  # a 16-bit out over fp32 y
    assert chk(z=None) < 0
    assert chk(out=None) == 0  # the backward's arguments carry no out
    assert lib.rp_mixer_out_fwd(ctypes.byref(_mixer_args(out=None)), None) < 0
    assert "NULL out" in lib.rp_last_error().decode()
    assert chk(u=0x3000001) < 0 and "misaligned" in lib.rp_last_error().decode()
    assert chk(u_sl=-1) < 0
    assert chk(out=0x3000000 + 64) < 0 and "overlaps" in lib.rp_last_error().decode()
    assert chk(out=0x1000000 + 4) < 0  # partly over y
    assert chk(D=1 << 31) < 0
    # nothing to do: no pointers needed
    assert chk(B=0, y=None, u=None, z=None, Dskip=None, out=None) == 0


def test_mixer_out_workspace(lib):
    a = _mixer_args()
    wb = lib.rp_mixer_out_work_bytes(ctypes.byref(a))
    assert wb > 0 and wb % 256 == 0
    # row groups x channels float64 partials; a fixed function of the shape
    assert wb >= 320 * 8 and wb == lib.rp_mixer_out_work_bytes(ctypes.byref(_mixer_args()))
    assert lib.rp_mixer_out_work_bytes(ctypes.byref(_mixer_args(k_skip=0))) < 0


def test_mixer_out_bwd_rules(lib):
    a = _mixer_args(dtype_u=_lib.RP_F32, dtype_z=_lib.RP_F32, z_sb=64 * 320, z_sl=320,
                    z=0x4000000)
    n = 4 * 64 * 320 * 4
    wb = lib.rp_mixer_out_work_bytes(ctypes.byref(a))
    base = dict(dout=0x6000000, dy=0x7000000, du=0x8000000, dz=0x9000000, dD=0xa000000,
                work=0xb000000, work_bytes=wb)
    bwd = lambda **kw: lib.rp_mixer_out_bwd(ctypes.byref(a), ctypes.byref(
        _lib.MixerOutGrad(**{**base, **kw})), None)
    # each failure below is caught on the host, before any launch
    assert bwd(work_bytes=wb - 8) == -4
    assert bwd(work=0xb000000 + 16) == -4
    assert bwd(du=0x9000000 + 128) < 0 and "overlap" in lib.rp_last_error().decode()
    assert bwd(dz=0x3000000) < 0 and "overlaps an input" in lib.rp_last_error().decode()
    assert bwd(dD=None) < 0
    assert bwd(dy=None) < 0
    assert n < 0x1000000


def _bcnorm_args(**kw):
    a = _lib.BcNormArgs()
    a.T, a.N, a.P = 1000, 40, 4
    a.dtype_x, a.normalize, a.eps = _lib.RP_BF16, 1, 1e-5
    a.B_raw, a.B_sr = 0x1000000 + 2 * 7, 7 + 320
    a.C_raw, a.C_sr = 0x1000000 + 2 * (7 + 160), 7 + 320
    a.wB, a.wC = 0x2000000, 0x2001000
    a.Bc, a.Cc = 0x3000000, 0x3100000
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def test_bcnorm_check(lib):
    chk = lambda **kw: lib.rp_bcnorm_check(ctypes.byref(_bcnorm_args(**kw)))
    assert chk() == 0
    assert chk(P=9) == -2 and chk(N=129) == -2
    assert chk(N=0) < 0 and chk(T=-1) < 0
    assert chk(dtype_x=5) < 0
    assert chk(normalize=2) < 0 and chk(reserved=1) < 0
    assert chk(wB=None) < 0 and "wB" in lib.rp_last_error().decode()
    assert chk(normalize=0, wB=None, wC=None) == 0  # plain p-sum: no weights
    assert chk(B_sr=100) < 0 and "row stride" in lib.rp_last_error().decode()
    assert chk(B_raw=0x1000001) < 0
    assert chk(eps=-1.0) < 0
    assert chk(T=0, B_raw=None, C_raw=None) == 0
    # outputs over an input are refused before any launch
    assert lib.rp_bcnorm_fwd(ctypes.byref(_bcnorm_args(Bc=0x1000000)), None) < 0
    assert "overlap" in lib.rp_last_error().decode()


def test_bcnorm_workspace(lib):
    a = _bcnorm_args()
    wb = lib.rp_bcnorm_work_bytes(ctypes.byref(a))
    assert wb > 0 and wb % 256 == 0 and wb >= 2 * 160 * 8
    g = _lib.BcNormGrad(dBc=0x4000000, dCc=0x4100000, dB_raw=0x5000000, dC_raw=0x5200000,
                        dwB=0x6000000, dwC=0x6001000, work=0x7000000, work_bytes=wb - 256)
    assert lib.rp_bcnorm_bwd(ctypes.byref(a), ctypes.byref(g), None) == -4


def test_rmsnorm_check(lib):
    def chk(**kw):
        a = _lib.RmsNormArgs(rows=16, d=512, eps=1e-5, x=0x100000, x_sr=512, w=0x200000,
                             out=0x300000)
        for k, v in kw.items():
            setattr(a, k, v)
        return lib.rp_rmsnorm_check(ctypes.byref(a))
    assert chk() == 0
    assert chk(x_sr=511) < 0
    assert chk(eps=-1.0) < 0
    assert chk(out=0x100000 + 64) < 0 and "overlaps" in lib.rp_last_error().decode()
    add = dict(add=0x400000, add_sr=1024, dtype_add=_lib.RP_BF16, x_out=0x500000)
    assert chk(**add) == 0
    assert chk(**{**add, "x_out": None}) < 0
    assert chk(**{**add, "dtype_add": 4}) < 0
    assert chk(**{**add, "x_out": 0x400000}) < 0
    assert chk(rows=0, x=None, w=None, out=None) == 0


def test_ply_topk_check(lib):
    def chk(**kw):
        a = _lib.PlyTopkArgs(R=4096, V=8192, k=8, dtype_logits=_lib.RP_F32, logits=0x1000000,
                             logits_sr=8192, values=0x100, out=0x10000000, out_sr=17)
        for k, v in kw.items():
            setattr(a, k, v)
        return lib.rp_ply_topk_check(ctypes.byref(a))
    assert chk() == 0
    assert chk(k=0) < 0 and chk(k=17) < 0 and chk(k=16, out_sr=33) == 0
    assert chk(out_sr=16) < 0
    assert chk(V=0) < 0 and chk(logits_sr=8191) < 0
    assert chk(dtype_logits=5) < 0
    assert chk(dtype_logits=_lib.RP_BF16, logits=0x1000001) < 0
    assert chk(out=0x1000000 + 64) < 0 and "overlaps" in lib.rp_last_error().decode()
    assert chk(R=0, logits=None, out=None) == 0


def test_ply_gather_check(lib):
    def chk(**kw):
        a = _lib.PlyGatherArgs(R=64, V=8192, M=40, dtype_logits=_lib.RP_BF16, logits=0x1000000,
                               logits_sr=8192, tokens=0x100000, tokens_sr=40, out=0x200000,
                               out_sr=40)
        for k, v in kw.items():
            setattr(a, k, v)
        return lib.rp_ply_gather_check(ctypes.byref(a))
    assert chk() == 0
    assert chk(reserved=1) < 0
    assert chk(tokens_sr=39) < 0 and chk(out_sr=39) < 0
    assert chk(tokens=0x100002) < 0
    assert chk(out=0x100000) < 0
    assert chk(M=0, tokens=None, out=None) == 0


def test_step_bcnorm_rules(lib):
    """rp_step_bcnorm validates both argument sets and their agreement before
    any launch: T = R, the same d_state, and the step's B / C rows being the
    BCNorm outputs with row stride N."""
    a = _step_args(Bc=0x3000000, Cc=0x3100000)
    bn = _bcnorm_args(T=16, N=20, P=2, B_sr=40, C_sr=40, B_raw=0x1000000, C_raw=0x1000100,
                      Bc=0x3000000, Cc=0x3100000)
    assert lib.rp_bcnorm_check(ctypes.byref(bn)) == 0
    call = lambda a, bn: lib.rp_step_bcnorm(ctypes.byref(a), ctypes.byref(bn), None)
    assert call(a, _bcnorm_args(**{**{"T": 17, "N": 20, "P": 2, "B_sr": 40, "C_sr": 40},
                                   "Bc": 0x3000000, "Cc": 0x3100000})) < 0
    assert "T must be R" in lib.rp_last_error().decode()
    assert call(a, _bcnorm_args(T=16, N=10, P=4, B_sr=40, C_sr=40, Bc=0x3000000,
                                Cc=0x3100000)) < 0
    assert call(_step_args(Bc=0x3000000, Cc=0x3200000), bn) < 0
    assert "bn->Bc" in lib.rp_last_error().decode()
    assert call(a, _bcnorm_args(T=16, N=20, P=2, B_sr=39, C_sr=40, Bc=0x3000000,
                                Cc=0x3100000)) < 0  # BCNorm's own rules
    assert lib.rp_step_bcnorm(ctypes.byref(a), None, None) < 0
    # nothing to do, so nothing is launched
    assert call(_step_args(R=0, Bc=0x3000000, Cc=0x3100000),
                _bcnorm_args(T=0, N=20, P=2, B_sr=40, C_sr=40, Bc=0x3000000, Cc=0x3100000)) == 0
