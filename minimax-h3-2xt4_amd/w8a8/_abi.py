"""ctypes binding of libw8a8.so (the C ABI declared in include/w8a8.h).

The library is loaded after torch so that it shares torch's HIP runtime
(both resolve the soname libamdhip64.so.7), hence the same streams. There is
no fallback: a missing library or a failing call raises.
"""
import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (must be loaded before the library; see above)

LIB_PATH = Path(__file__).resolve().parent / 'libw8a8.so'

OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_LAUNCH = 0, 1, 2, 3
F16, BF16, F32, I32, I8 = 1, 2, 3, 4, 5
EPI_INT32, EPI_ROW, EPI_COLUMN = 0, 1, 2
ABI_VERSION = 13

_c = ctypes
_p = ctypes.c_void_p


class QuantArgs(ctypes.Structure):
    _fields_ = [('struct_size', _c.c_uint32), ('x_dtype', _c.c_int32), ('x', _p), ('ldx', _c.c_int64),
                ('rows', _c.c_int64), ('cols', _c.c_int64), ('convrot', _c.c_int32),
                ('round_rotated', _c.c_int32), ('row_max', _p), ('q', _p), ('ldq', _c.c_int64),
                ('scale', _p), ('stream', _p), ('row_max_out', _p), ('convrot_signs', _p)]


class SwigluArgs(ctypes.Structure):
    _fields_ = [('struct_size', _c.c_uint32), ('x_dtype', _c.c_int32), ('x', _p), ('ldx', _c.c_int64),
                ('rows', _c.c_int64), ('width', _c.c_int64), ('row_max', _p), ('row_max_out', _p),
                ('group_max', _p), ('q', _p), ('ldq', _c.c_int64), ('scale', _p), ('stream', _p),
                ('convrot_signs', _p)]


class RopeEpilogue(ctypes.Structure):
    _fields_ = [('heads', _c.c_int32), ('rot_dim', _c.c_int32), ('freq_dtype', _c.c_int32), ('eps', _c.c_float),
                ('freq_layout', _c.c_int32), ('reserved', _c.c_int32), ('freqs', _p), ('q_gain', _p), ('k_gain', _p)]


class GemmArgs(ctypes.Structure):
    _fields_ = [('struct_size', _c.c_uint32), ('epilogue', _c.c_int32), ('a', _p), ('lda', _c.c_int64),
                ('b', _p), ('ldb', _c.c_int64), ('m', _c.c_int64), ('n', _c.c_int64), ('k', _c.c_int64),
                ('row_scale', _p), ('col_scale', _p), ('col_scale_stride', _c.c_int64), ('bias', _p),
                ('bias_dtype', _c.c_int32), ('out_dtype', _c.c_int32), ('residual', _p),
                ('ldr', _c.c_int64), ('gate', _p), ('gate_labels', _p), ('ldg', _c.c_int64), ('out', _p),
                ('ldc', _c.c_int64), ('workspace', _p),
                ('workspace_bytes', _c.c_int64), ('rope', ctypes.POINTER(RopeEpilogue)), ('stream', _p)]


class DequantArgs(ctypes.Structure):
    _fields_ = [('struct_size', _c.c_uint32), ('epilogue', _c.c_int32), ('acc', _p), ('ldacc', _c.c_int64),
                ('m', _c.c_int64), ('n', _c.c_int64), ('row_scale', _p), ('col_scale', _p),
                ('col_scale_stride', _c.c_int64), ('bias', _p), ('bias_dtype', _c.c_int32),
                ('out_dtype', _c.c_int32), ('residual', _p), ('ldr', _c.c_int64), ('gate', _p),
                ('gate_labels', _p), ('ldg', _c.c_int64), ('out', _p), ('ldc', _c.c_int64), ('stream', _p)]


class NormArgs(ctypes.Structure):
    _fields_ = [('struct_size', _c.c_uint32), ('x_dtype', _c.c_int32), ('x', _p), ('ldx', _c.c_int64),
                ('rows', _c.c_int64), ('cols', _c.c_int64), ('weight', _p), ('mod_shift', _p),
                ('mod_scale', _p), ('ld_mod', _c.c_int64), ('mod_rows', _c.c_int32), ('eps', _c.c_float),
                ('labels', _p), ('y', _p), ('ldy', _c.c_int64), ('convrot', _c.c_int32),
                ('round_rotated', _c.c_int32), ('q', _p), ('ldq', _c.c_int64), ('q_scale', _p), ('stream', _p),
                ('convrot_signs', _p)]


class RmsRopeArgs(ctypes.Structure):
    _fields_ = [('struct_size', _c.c_uint32), ('in_dtype', _c.c_int32), ('packed', _p), ('ldp', _c.c_int64),
                ('rows', _c.c_int64), ('heads', _c.c_int32), ('dim', _c.c_int32), ('rot_dim', _c.c_int32),
                ('freq_dtype', _c.c_int32), ('freqs', _p), ('q_gain', _p), ('k_gain', _p), ('eps', _c.c_float),
                ('out_dtype', _c.c_int32), ('q_out', _p), ('k_out', _p), ('stream', _p)]


class AttnPrepareArgs(ctypes.Structure):
    _fields_ = [('struct_size', _c.c_uint32), ('in_dtype', _c.c_int32), ('q', _p), ('k', _p), ('v', _p),
                ('b', _c.c_int64), ('h', _c.c_int64), ('nq', _c.c_int64), ('nk', _c.c_int64), ('d', _c.c_int32),
                ('sm_scale', _c.c_float), ('q_strides', _c.c_int64 * 3), ('k_strides', _c.c_int64 * 3),
                ('v_strides', _c.c_int64 * 3), ('q8', _p), ('qs', _p), ('k8', _p), ('ks', _p), ('vt8', _p),
                ('vs', _p), ('vsum', _p), ('workspace', _p), ('workspace_bytes', _c.c_int64), ('stream', _p)]


class AttentionArgs(ctypes.Structure):
    _fields_ = [('struct_size', _c.c_uint32), ('out_dtype', _c.c_int32), ('q8', _p), ('qs', _p), ('k8', _p),
                ('ks', _p), ('vt8', _p), ('vs', _p), ('vsum', _p), ('b', _c.c_int64), ('h', _c.c_int64), ('nq', _c.c_int64),
                ('nk', _c.c_int64), ('d', _c.c_int32), ('sm_scale', _c.c_float), ('out', _p),
                ('out_strides', _c.c_int64 * 3), ('stream', _p)]


# Argument structs in w8a8_struct_size() index order, with their entry points.
STRUCTS = (QuantArgs, SwigluArgs, GemmArgs, DequantArgs, NormArgs, RmsRopeArgs, AttnPrepareArgs, AttentionArgs)
STRUCT_ENTRY_POINTS = ('w8a8_quantize_rows', 'w8a8_swiglu_quantize', 'w8a8_gemm', 'w8a8_dequantize',
                       'w8a8_norm_quantize', 'w8a8_rms_rope', 'w8a8_attention_prepare', 'w8a8_attention')
ENTRY_POINTS = STRUCT_ENTRY_POINTS + ('w8a8_gemm_noalloc', 'w8a8_abi_version', 'w8a8_struct_size',
                                      'w8a8_last_error', 'w8a8_gemm_workspace_size',
                                      'w8a8_attention_workspace_size')
GEMM_SCRATCH_BYTES = 64 << 20   # W8A8_GEMM_SCRATCH_BYTES: the no-allocation GEMM's split-K scratch per GPU

_LIB = None


class W8A8Error(RuntimeError):
    """A libw8a8 entry point returned a non-zero status."""

    def __init__(self, fn, code, message):
        super().__init__(f'{fn} failed with status {code}: {message}')
        self.code = code


def load(path=None):
    """Load and verify libw8a8.so (ABI version and argument-struct sizes)."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise RuntimeError(f'{p} is missing: build it with python minimax-h3-2xt4_amd/build_lib.py '
                           '(there is no CPU fallback for the W8A8 path)')
    lib = ctypes.CDLL(os.fspath(p))
    lib.w8a8_abi_version.restype = _c.c_int
    lib.w8a8_struct_size.restype = _c.c_int64
    lib.w8a8_struct_size.argtypes = [_c.c_int32]
    lib.w8a8_last_error.restype = _c.c_char_p
    lib.w8a8_gemm_workspace_size.restype = _c.c_int64
    lib.w8a8_gemm_workspace_size.argtypes = [_c.c_int64, _c.c_int64, _c.c_int64]
    lib.w8a8_attention_workspace_size.restype = _c.c_int64
    lib.w8a8_attention_workspace_size.argtypes = [_c.c_int64, _c.c_int64, _c.c_int64]
    for name, st in zip(STRUCT_ENTRY_POINTS + ('w8a8_gemm_noalloc',), STRUCTS + (GemmArgs,)):
        fn = getattr(lib, name)
        fn.restype = _c.c_int
        fn.argtypes = [ctypes.POINTER(st)]
    if lib.w8a8_abi_version() != ABI_VERSION:
        raise RuntimeError(f'libw8a8 ABI {lib.w8a8_abi_version()} != {ABI_VERSION}')
    for i, st in enumerate(STRUCTS):
        if lib.w8a8_struct_size(i) != ctypes.sizeof(st):
            raise RuntimeError(f'{st.__name__}: library size {lib.w8a8_struct_size(i)} != '
                               f'binding size {ctypes.sizeof(st)}')
    if path is None:
        _LIB = lib
    return lib


def call(name, args):
    lib = load()
    args.struct_size = ctypes.sizeof(args)
    rc = getattr(lib, name)(ctypes.byref(args))
    if rc != OK:
        raise W8A8Error(name, rc, lib.w8a8_last_error().decode(errors='replace'))


def ptr(t):
    return None if t is None else t.data_ptr()


def stream_of(t):
    return torch.cuda.current_stream(t.device).cuda_stream


DTYPE_CODE = {torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32, torch.int32: I32, torch.int8: I8}
