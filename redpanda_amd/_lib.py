"""ctypes binding of libredpanda_hip.so (the C ABI in include/redpanda_hip.h).

The structures below mirror the header field for field.  `load()` opens the
in-tree library built by `redpanda_amd.build`; there is no fallback: a
missing library or a missing GPU raises, so nothing silently runs elsewhere.
"""

import ctypes
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libredpanda_hip.so")

ABI_VERSION = 13
RP_F32, RP_BF16, RP_F16 = 0, 1, 2
DTYPE_CODES = {torch.float32: RP_F32, torch.bfloat16: RP_BF16, torch.float16: RP_F16}
MAX_STATE = 128

_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_vp = ctypes.c_void_p


class ScanArgs(ctypes.Structure):
    _fields_ = [
        ("B", _i64), ("L", _i64), ("D", _i64), ("N", _i64), ("NR", _i64), ("NT", _i64),
        ("dtype_delta", _i32), ("dtype_u", _i32), ("dtype_B", _i32), ("dtype_C", _i32),
        ("bidirectional", _i32), ("delta_softplus", _i32),
        ("delta", _vp), ("delta_sb", _i64), ("delta_sl", _i64),
        ("u", _vp), ("u_sb", _i64), ("u_sl", _i64),
        ("Bc", _vp), ("Bc_sb", _i64), ("Bc_sl", _i64),
        ("Cc", _vp), ("Cc_sb", _i64), ("Cc_sl", _i64),
        ("A_real", _vp), ("A_imag", _vp), ("track", _vp), ("h0", _vp), ("beta0", _vp),
        ("grad_in_storage", _i32),
    ]


class ScanFwdOut(ctypes.Structure):
    _fields_ = [("y", _vp), ("ckpt", _vp), ("h_last", _vp), ("beta_last", _vp)]


class ScanBwdIO(ctypes.Structure):
    _fields_ = [
        ("dy", _vp), ("ckpt", _vp), ("dh_last", _vp), ("dbeta_last", _vp),
        ("d_delta", _vp), ("d_u", _vp), ("d_Bc", _vp),
        ("d_Cc", _vp), ("d_A_real", _vp), ("d_A_imag", _vp), ("d_track", _vp),
        ("d_h0", _vp), ("d_beta0", _vp), ("work", _vp), ("work_bytes", _i64),
    ]


class StepArgs(ctypes.Structure):
    _fields_ = [
        ("R", _i64), ("D", _i64), ("N", _i64), ("NR", _i64), ("NT", _i64),
        ("delta", _vp), ("delta_sr", _i64), ("u", _vp), ("u_sr", _i64),
        ("Bc", _vp), ("Bc_sr", _i64), ("Cc", _vp), ("Cc_sr", _i64),
        ("h_in", _vp), ("beta_in", _vp), ("A_real", _vp), ("A_imag", _vp), ("track", _vp),
        ("Dskip", _vp), ("h_out", _vp), ("beta_out", _vp), ("y", _vp),
        ("broadcast_state", _i32), ("delta_softplus", _i32),
        ("beta_rank1", _i32), ("reserved", _i32),
        ("z", _vp), ("z_sr", _i64), ("dtype_z", _i32), ("reserved2", _i32),
    ]


class MixerOutArgs(ctypes.Structure):
    _fields_ = [
        ("B", _i64), ("L", _i64), ("D", _i64),
        ("k_skip", _i32), ("dtype_u", _i32), ("dtype_z", _i32), ("dtype_out", _i32),
        ("y", _vp), ("u", _vp), ("u_sb", _i64), ("u_sl", _i64),
        ("z", _vp), ("z_sb", _i64), ("z_sl", _i64), ("Dskip", _vp), ("out", _vp),
    ]


class MixerOutGrad(ctypes.Structure):
    _fields_ = [
        ("dout", _vp), ("dy", _vp), ("du", _vp), ("dz", _vp), ("dD", _vp),
        ("work", _vp), ("work_bytes", _i64),
    ]


class BcNormArgs(ctypes.Structure):
    _fields_ = [
        ("T", _i64), ("N", _i64), ("P", _i64),
        ("dtype_x", _i32), ("normalize", _i32), ("eps", ctypes.c_float), ("reserved", _i32),
        ("B_raw", _vp), ("B_sr", _i64), ("C_raw", _vp), ("C_sr", _i64),
        ("wB", _vp), ("wC", _vp), ("Bc", _vp), ("Cc", _vp),
    ]


class BcNormGrad(ctypes.Structure):
    _fields_ = [
        ("dBc", _vp), ("dCc", _vp), ("dB_raw", _vp), ("dC_raw", _vp),
        ("dwB", _vp), ("dwC", _vp), ("work", _vp), ("work_bytes", _i64),
    ]


class RmsNormArgs(ctypes.Structure):
    _fields_ = [
        ("rows", _i64), ("d", _i64), ("dtype_add", _i32), ("eps", ctypes.c_float),
        ("x", _vp), ("x_sr", _i64), ("add", _vp), ("add_sr", _i64),
        ("w", _vp), ("x_out", _vp), ("out", _vp),
    ]


class PlyTopkArgs(ctypes.Structure):
    _fields_ = [
        ("R", _i64), ("V", _i64), ("k", _i32), ("dtype_logits", _i32),
        ("logits", _vp), ("logits_sr", _i64), ("values", _vp), ("out", _vp), ("out_sr", _i64),
    ]


class PlyGatherArgs(ctypes.Structure):
    _fields_ = [
        ("R", _i64), ("V", _i64), ("M", _i64), ("dtype_logits", _i32), ("reserved", _i32),
        ("logits", _vp), ("logits_sr", _i64), ("tokens", _vp), ("tokens_sr", _i64),
        ("out", _vp), ("out_sr", _i64),
    ]


# Every symbol include/redpanda_hip.h declares, with its ctypes signature.
SIGNATURES = {
    "rp_abi_version": (ctypes.c_int, []),
    "rp_last_error": (ctypes.c_char_p, []),
    "rp_scan_check": (ctypes.c_int, [ctypes.POINTER(ScanArgs)]),
    "rp_scan_ckpt_bytes": (_i64, [ctypes.POINTER(ScanArgs)]),
    "rp_scan_bwd_work_bytes": (_i64, [ctypes.POINTER(ScanArgs)]),
    "rp_scan_fwd": (ctypes.c_int, [ctypes.POINTER(ScanArgs), ctypes.POINTER(ScanFwdOut), _vp]),
    "rp_scan_bwd": (ctypes.c_int, [ctypes.POINTER(ScanArgs), ctypes.POINTER(ScanBwdIO), _vp]),
    "rp_scan_bwd_noalloc": (ctypes.c_int, [ctypes.POINTER(ScanArgs), ctypes.POINTER(ScanBwdIO),
                                           _vp]),
    "rp_step_check": (ctypes.c_int, [ctypes.POINTER(StepArgs)]),
    "rp_step": (ctypes.c_int, [ctypes.POINTER(StepArgs), _vp]),
    "rp_bcnorm_check": (ctypes.c_int, [ctypes.POINTER(BcNormArgs)]),
    "rp_bcnorm_work_bytes": (_i64, [ctypes.POINTER(BcNormArgs)]),
    "rp_bcnorm_fwd": (ctypes.c_int, [ctypes.POINTER(BcNormArgs), _vp]),
    "rp_bcnorm_bwd": (ctypes.c_int, [ctypes.POINTER(BcNormArgs), ctypes.POINTER(BcNormGrad), _vp]),
    "rp_step_bcnorm": (ctypes.c_int, [ctypes.POINTER(StepArgs), ctypes.POINTER(BcNormArgs), _vp]),
    "rp_rmsnorm_check": (ctypes.c_int, [ctypes.POINTER(RmsNormArgs)]),
    "rp_rmsnorm_fwd": (ctypes.c_int, [ctypes.POINTER(RmsNormArgs), _vp]),
    "rp_softplus": (ctypes.c_int, [_vp, _vp, _i64, _vp]),
    "rp_ply_topk_check": (ctypes.c_int, [ctypes.POINTER(PlyTopkArgs)]),
    "rp_ply_topk": (ctypes.c_int, [ctypes.POINTER(PlyTopkArgs), _vp]),
    "rp_ply_gather_check": (ctypes.c_int, [ctypes.POINTER(PlyGatherArgs)]),
    "rp_ply_gather": (ctypes.c_int, [ctypes.POINTER(PlyGatherArgs), _vp]),
    "rp_mixer_out_check": (ctypes.c_int, [ctypes.POINTER(MixerOutArgs)]),
    "rp_mixer_out_work_bytes": (_i64, [ctypes.POINTER(MixerOutArgs)]),
    "rp_mixer_out_fwd": (ctypes.c_int, [ctypes.POINTER(MixerOutArgs), _vp]),
    "rp_mixer_out_bwd": (ctypes.c_int, [ctypes.POINTER(MixerOutArgs),
                                        ctypes.POINTER(MixerOutGrad), _vp]),
}

_LIB = None


def open_library(path=LIB_PATH):
    """dlopen the library and attach signatures (no GPU needed)."""
    if not os.path.exists(path):
        raise RuntimeError(
            f"redpanda_amd: HIP library not built ({path} missing); run "
            "`python -m redpanda_amd.build`")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.rp_abi_version() != ABI_VERSION:
        raise RuntimeError(f"redpanda_amd: ABI {lib.rp_abi_version()} != {ABI_VERSION}")
    return lib


def hip_runtimes_mapped():
    """Distinct HIP runtime files mapped into this process (Linux)."""
    try:
        with open("/proc/self/maps") as fh:
            paths = {line.split()[-1] for line in fh if "libamdhip64" in line}
    except OSError:
        return set()
    return {os.path.realpath(p) for p in paths}


def load():
    """The library, for use on a GPU.  Raises if there is no GPU or no library.

    The library's DT_NEEDED libamdhip64.so.7 must resolve to the runtime torch
    already loaded (same soname), so torch's streams and allocations are valid
    handles inside it; a second runtime in the process is an error.
    """
    global _LIB
    if _LIB is None:
        if not torch.cuda.is_available():
            raise RuntimeError("redpanda_amd: the HIP kernels need a ROCm GPU (none visible)")
        torch.cuda.init()
        lib = open_library()
        rts = hip_runtimes_mapped()
        if len(rts) > 1:
            raise RuntimeError(f"redpanda_amd: two HIP runtimes in one process: {sorted(rts)}")
        _LIB = lib
    return _LIB


def check(status, lib=None):
    if status != 0:
        lib = lib or _LIB
        msg = lib.rp_last_error().decode(errors="replace") if lib is not None else ""
        raise RuntimeError(f"redpanda_amd: status {status}: {msg}")


def ptr(t):
    return None if t is None else t.data_ptr()


def stream_of(device):
    return torch.cuda.current_stream(device).cuda_stream
