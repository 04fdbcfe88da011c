"""ctypes binding of libapexw_hip.so (the C ABI declared in include/apexw_hip.h).

The library is built in-tree by ``apexw_amd._build``.  There is no fallback: if
the library is missing or was built for another ABI version, every entry point
raises.  Struct layouts below mirror the header field for field; the numpy
dtypes are the same layouts used to build device-resident tables in bulk.
"""

import ctypes
import os

import numpy as np

from ._build import LIB_PATH

ABI_VERSION = 24

# dtype codes
F32, BF16, F16, U8, I8 = 0, 1, 2, 3, 4

# apexw_tensor.flags
PDT_SHIFT, GDT_SHIFT, MDT_SHIFT, VDT_SHIFT = 0, 2, 4, 6
FLAG_QUAD = 1 << 8
FLAG_WD = 1 << 9
FLAG_NF4 = 1 << 10
FLAG_GENERIC = 1 << 11
FLAG_DENSE = 1 << 12
FLAG_SCALAR = 1 << 13
FLAG_FACTORED = 1 << 14
FLAG_M6 = 1 << 15
FLAG_GC = 1 << 16
FLAG_ULTRA = 1 << 17
FLAG_VSCALE = 1 << 18

COMPACT_UNIT = 2048

MODE_COLD, MODE_REPLAY, MODE_NATIVE, MODE_SINGLE = 0, 1, 2, 3

HP_SR = 1 << 0
HP_SR_V = 1 << 1
HP_SANITIZE = 1 << 2
HP_CLIP = 1 << 3
HP_LERP_HI = 1 << 4
HP_LOOK_HI = 1 << 5
HP_UNSCALE = 1 << 6
HP_FV_SANITIZE = 1 << 7
HP_AMP = 1 << 8
HP_NESTEROV = 1 << 9
HP_CAUTIOUS = 1 << 10
HP_AMSGRAD = 1 << 11
HP_LION = 1 << 12
HP_SLOW = 1 << 13
HP_LERP3_HI = 1 << 14
HP_GRAD_DTYPES = 1 << 15

STATUS = {0: "ok", 1: "invalid argument", 2: "unsupported dtype combination", 3: "launch failed",
          4: "misaligned pointer", 5: "exceeds the fixed workspace of the allocation-free entry point"}
ERR_SIZE = 5
NOALLOC_CLIP_MAX_UNITS = 1 << 23
NOALLOC_CLIP_MAX_TENSORS = 1 << 17

TENSOR_DTYPE = np.dtype([
    ("p", np.uint64), ("g", np.uint64), ("m", np.uint64), ("v", np.uint64),
    ("m_scale", np.uint64), ("v_scale", np.uint64), ("n", np.int64),
    ("flags", np.uint32), ("block", np.uint32),
])
UNIT_DTYPE = np.dtype([("tensor", np.uint32), ("unit", np.uint32)])
assert TENSOR_DTYPE.itemsize == 64 and UNIT_DTYPE.itemsize == 8


class Tensor(ctypes.Structure):
    _fields_ = [("p", ctypes.c_void_p), ("g", ctypes.c_void_p), ("m", ctypes.c_void_p), ("v", ctypes.c_void_p),
                ("m_scale", ctypes.c_void_p), ("v_scale", ctypes.c_void_p), ("n", ctypes.c_int64),
                ("flags", ctypes.c_uint32), ("block", ctypes.c_uint32)]


class StateLayout(ctypes.Structure):
    """apexw_state_layout: one parameter's moment buffers, for conversion between precision modes."""
    _fields_ = [("m", ctypes.c_void_p), ("v", ctypes.c_void_p), ("m_scale", ctypes.c_void_p),
                ("v_scale", ctypes.c_void_p), ("n", ctypes.c_int64), ("kind", ctypes.c_uint32),
                ("flags", ctypes.c_uint32), ("block", ctypes.c_uint32), ("reserved", ctypes.c_uint32)]


STATE_DENSE, STATE_Q8 = 0, 1
assert ctypes.sizeof(StateLayout) == 56


class HParams(ctypes.Structure):
    _fields_ = [("beta1", ctypes.c_float), ("one_minus_beta1", ctypes.c_float),
                ("beta2", ctypes.c_float), ("one_minus_beta2", ctypes.c_float),
                ("wd_factor", ctypes.c_float), ("step_size", ctypes.c_float),
                ("eps_scaled", ctypes.c_float), ("eps", ctypes.c_float),
                ("lerp_coef", ctypes.c_float), ("look_coef", ctypes.c_float),
                ("bc2_sqrt", ctypes.c_float), ("gain_hi", ctypes.c_float), ("gain_lo", ctypes.c_float),
                ("clip_coef", ctypes.c_void_p), ("seed", ctypes.c_uint64), ("step", ctypes.c_uint32),
                ("mode", ctypes.c_uint32), ("flags", ctypes.c_uint32), ("grad_inv_scale", ctypes.c_float),
                ("amp", ctypes.c_void_p), ("rows", ctypes.c_void_p), ("counts", ctypes.c_void_p),
                ("max_v", ctypes.c_void_p), ("beta3", ctypes.c_float), ("one_minus_beta3", ctypes.c_float),
                ("lerp3_coef", ctypes.c_float), ("slow_ratio", ctypes.c_float), ("slow", ctypes.c_void_p)]


assert ctypes.sizeof(HParams) == 144
# apexw_row_means: grad centralization's row means of one 8-bit / ultra descriptor
ROW_MEANS_DTYPE = np.dtype([("means", np.uint64), ("row_len", np.int64)])


# apexw_amp_launch: one launch's host inputs to apexw_amp_prepare; apexw_amp_dyn: its device output
AMP_LAUNCH_DTYPE = np.dtype([("lr", np.float64), ("beta1", np.float64), ("beta2", np.float64), ("eps", np.float64),
                             ("step", np.float64), ("kind", np.uint32), ("reserved", np.uint32)])
assert AMP_LAUNCH_DTYPE.itemsize == 48
# apexw_check_launch kinds
LAUNCH_COMPACT, LAUNCH_Q8, LAUNCH_FACTORED, LAUNCH_ULTRA, LAUNCH_CAUTIOUS = 0, 1, 4, 5, 6

AMP_DYN_BYTES = 32
AMP_MAX_LAUNCHES = 16


# apexw_gemm_problem: one product of a grouped launch
GEMM_PROBLEM_DTYPE = np.dtype([
    ("a", np.uint64), ("b", np.uint64), ("et", np.uint64), ("c", np.uint64), ("ct", np.uint64),
    ("m", np.int32), ("n", np.int32), ("k", np.int32), ("lda", np.int32), ("ldb", np.int32), ("lde", np.int32),
    ("ldc", np.int32), ("ldct", np.int32), ("alpha", np.float32), ("beta", np.float32),
    ("flags", np.uint32), ("reserved", np.uint32),
    ("p", np.uint64), ("p_dtype", np.int32), ("p_rows", np.int32), ("p_cols", np.int32),
    ("wd_factor", np.float32), ("neg_lr", np.float32), ("reserved2", np.uint32),
])
assert GEMM_PROBLEM_DTYPE.itemsize == 120
_GEMM_APPLY_ZERO = (0, 0, 0, 0, 0.0, 0.0, 0)


def gemm_problems(rows):
    """A host table of GEMM_PROBLEM_DTYPE from tuples: the 17 product fields (a .. reserved),
    optionally followed by the 7 fields of a fused Muon update (p .. reserved2)."""
    return np.array([tuple(r) if len(r) == 24 else tuple(r) + _GEMM_APPLY_ZERO for r in rows],
                    dtype=GEMM_PROBLEM_DTYPE)
# apexw_grad_prep: one grad of a preparation launch (sanitize / unscale / centralize)
GRAD_PREP_DTYPE = np.dtype([("g", np.uint64), ("out", np.uint64), ("n", np.int64), ("row_len", np.int64),
                            ("dtype", np.uint32), ("reserved", np.uint32)])
assert GRAD_PREP_DTYPE.itemsize == 40
GRAD_PREP_CHUNK = 2048
# apexw_fv_tensor: one factored-v tensor of a group
FV_TENSOR_DTYPE = np.dtype([("tensor", np.uint32), ("rows", np.int32), ("cols", np.int32), ("flags", np.uint32),
                            ("ws", np.int64), ("band0", np.int32), ("cb0", np.int32)])
assert FV_TENSOR_DTYPE.itemsize == 32
FV_SUM_COLS = 1
FV_BAND_ROWS = 32
FV_UNIT_RANGES = 9   # (bf16, fp32, fp16 parameters) x (INT8, 6-bit, 16-bit m)

GEMM_SYM, GEMM_B_KN, GEMM_ADD_B, GEMM_APPLY, GEMM_APPLY_T, GEMM_APPLY_WD, GEMM_PANEL = 1, 2, 4, 8, 16, 32, 64
GEMM_OUT_C, GEMM_OUT_CT, GEMM_ADD, GEMM_KIND_NN, GEMM_KIND_PANEL = 1, 2, 4, 8, 16
LAYOUT_ROWS, LAYOUT_PANEL = 0, 1   # Newton-Schulz work matrices: row-major or 32 x 32 panels
GEMM_MAX_PROBLEMS = 256
GEMM_QUEUES = 8

_vp, _i32, _i64, _f32, _u32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_uint32
_HP = ctypes.POINTER(HParams)

# name -> (restype, argtypes); every symbol the header declares
SIGNATURES = {
    "apexw_abi_version": (ctypes.c_int, []),
    "apexw_check_tensor": (ctypes.c_int, [ctypes.POINTER(Tensor), _i32]),
    "apexw_check_launch": (ctypes.c_int, [_i32, _i32, _i64, _i64, _i64, _HP]),
    "apexw_compact_step": (ctypes.c_int, [_vp, _i32, _vp, _i64, _HP, _vp]),
    "apexw_ultra_step": (ctypes.c_int, [_vp, _i32, _vp, _i64, _HP, _vp]),
    "apexw_q8_step": (ctypes.c_int, [_vp, _i32, _vp, _i64, _i64, _i64, _HP, _vp]),
    "apexw_q8_cautious_count": (ctypes.c_int, [_vp, _i32, _vp, _i64, _HP, _vp]),
    "apexw_compact_cautious_count": (ctypes.c_int, [_vp, _i32, _vp, _i64, _HP, _vp]),
    "apexw_grad_clip_coef": (ctypes.c_int, [_vp, _i32, _vp, _i64, _i64, _vp, _vp, _vp, _f32, _f32, _u32, _vp, _vp, _vp,
                                            _vp]),
    "apexw_grad_clip_coef_noalloc": (ctypes.c_int, [_vp, _i32, _vp, _i64, _i64, _vp, _f32, _f32, _u32, _vp, _vp, _vp]),
    "apexw_gemm_nt_bf16": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                                          _i32, _i64, _i64, _i64, _i64, _i64, _f32, _f32, _vp]),
    "apexw_check_grad_prep": (ctypes.c_int, [_vp]),
    "apexw_check_row_means": (ctypes.c_int, [_vp]),
    "apexw_grad_prep_units": (ctypes.c_int64, [_vp]),
    "apexw_grad_prepare": (ctypes.c_int, [_vp, _i32, _vp, _i64, _f32, _u32, _vp, _vp]),
    "apexw_grad_row_means": (ctypes.c_int, [_vp, _i32, _vp, _i64, _f32, _u32, _vp, _vp]),
    "apexw_gemm_grouped_items": (ctypes.c_int64, [_vp, _i32]),
    "apexw_gemm_grouped_schedule": (ctypes.c_int, [_vp, _i32, _vp, _i64, _i32, ctypes.POINTER(ctypes.c_int64), _vp,
                                                   ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32)]),
    "apexw_gemm_nt_grouped": (ctypes.c_int, [_vp, _vp, _vp, _i32, _i32, _vp, _vp]),
    "apexw_muon_workspace_floats": (ctypes.c_int64, [_i64, _i64]),
    "apexw_muon_prepare": (ctypes.c_int, [_vp, _vp, _i32, _i64, _i64, _f32, _f32, _i32, _f32, _f32, _vp, _vp, _i64,
                                          _i64, _i32, _vp, _vp, _vp]),
    "apexw_muon_apply": (ctypes.c_int, [_vp, _i32, _vp, _i64, _i64, _i64, _i32, _i32, _f32, _i32, _f32, _vp, _vp]),
    "apexw_factored_layout": (ctypes.c_int64, [_vp, _i32, ctypes.POINTER(ctypes.c_int64),
                                               ctypes.POINTER(ctypes.c_int64)]),
    "apexw_factored_step": (ctypes.c_int, [_vp, _i32, _vp, _i32, _i64, _i64, _vp, _i64, _vp, _vp, _HP, _vp]),
    "apexw_muon_coordwise": (ctypes.c_int, [_vp, _vp, _i32, _vp, _i32, _i64, _f32, _f32, _i32, _f32, _f32, _i32,
                                             _f32, _vp, _vp]),
    "apexw_amp_prepare": (ctypes.c_int, [_vp, _vp, _vp, _i32, _vp, _i32, _vp, _vp]),
    "apexw_state_decode": (ctypes.c_int, [ctypes.POINTER(StateLayout), _vp, _vp, _vp]),
    "apexw_state_encode": (ctypes.c_int, [ctypes.POINTER(StateLayout), _vp, _vp, _vp]),
}

GEMM_TILE = 256
GEMM_KTILE = 64

_LIB = None


class ApexwError(RuntimeError):
    pass


def load(path=LIB_PATH):
    """Load the library once; raise if it is missing or has another ABI version."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(path):
        raise ApexwError(f"{path} is not built; run `python -m apexw_amd._build` (hipcc, gfx950)")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    ver = lib.apexw_abi_version()
    if ver != ABI_VERSION:
        raise ApexwError(f"libapexw_hip ABI {ver}, expected {ABI_VERSION}; rebuild")
    _LIB = lib
    return lib


def check(status, what):
    if status != 0:
        raise ApexwError(f"{what}: {STATUS.get(status, status)}")


def gemm_schedule(problems, cus_per_queue=0):
    """Validate a host table of GEMM_PROBLEM_DTYPE rows and build its grouped-launch
    tile queues: returns (items uint32[n_items], queue_offsets int32[GEMM_QUEUES + 1],
    n_workgroups, kind).  cus_per_queue > 0 (the CUs of one XCD) lets the last
    tiles of a queue split into 128-row halves (item bits 22-23)."""
    lib = load()
    problems = np.ascontiguousarray(problems, dtype=GEMM_PROBLEM_DTYPE)
    n_tiles = int(lib.apexw_gemm_grouped_items(problems.ctypes.data, len(problems)))
    if n_tiles < 0:
        check(-n_tiles, "apexw_gemm_grouped_items")
    items = np.empty(max(2 * n_tiles, 1), dtype=np.uint32)
    offsets = np.empty(GEMM_QUEUES + 1, dtype=np.int32)
    n_items, n_wg, kind = ctypes.c_int64(0), ctypes.c_int32(0), ctypes.c_int32(0)
    check(lib.apexw_gemm_grouped_schedule(problems.ctypes.data, len(problems), items.ctypes.data, len(items),
                                          int(cus_per_queue), ctypes.byref(n_items), offsets.ctypes.data,
                                          ctypes.byref(n_wg), ctypes.byref(kind)),
          "apexw_gemm_grouped_schedule")
    return items[:n_items.value].copy(), offsets, n_wg.value, kind.value


def cus_per_queue(device):
    """CUs of one XCD of `device` (its CU count over the grouped launch's queues)."""
    import torch
    return max(1, torch.cuda.get_device_properties(device).multi_processor_count // GEMM_QUEUES)
