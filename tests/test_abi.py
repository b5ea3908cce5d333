"""The C ABI library on the CPU: it loads, exports every symbol the header
declares, agrees on struct layouts, and rejects invalid arguments before any
launch (nothing here runs device code)."""
import ctypes
import re
from pathlib import Path

import pytest
import torch  # noqa: F401  (loaded first: the library shares torch's HIP runtime)

from w8a8 import _abi

HEADER = Path(__file__).resolve().parents[1] / 'include' / 'w8a8.h'


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r'^\s*(?:int|int64_t|const char\*)\s+(w8a8_\w+)\s*\(', text, re.M)))


def test_header_declares_the_entry_points():
    assert declared_functions() == sorted(_abi.ENTRY_POINTS)


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_abi.LIB_PATH))
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_version_and_struct_sizes():
    lib = _abi.load()
    assert lib.w8a8_abi_version() == _abi.ABI_VERSION
    for i, st in enumerate(_abi.STRUCTS):
        assert lib.w8a8_struct_size(i) == ctypes.sizeof(st)
    assert lib.w8a8_struct_size(99) == -1
    # header field order: sizes computed from the C declaration
    assert [ctypes.sizeof(s) for s in _abi.STRUCTS] == [104, 104, 192, 144, 152, 104, 224, 144]
    assert ctypes.sizeof(_abi.RopeEpilogue) == 48   # static_assert'ed in the library too


def _expect_invalid(name, args, fragment):
    lib = _abi.load()
    rc = getattr(lib, name)(ctypes.byref(args))
    assert rc == _abi.ERR_INVALID
    assert fragment in lib.w8a8_last_error().decode()


def test_struct_size_mismatch_rejected():
    a = _abi.QuantArgs(struct_size=12, x_dtype=_abi.F16)
    _expect_invalid('w8a8_quantize_rows', a, 'struct_size')


def test_quantize_argument_checks():
    base = dict(struct_size=ctypes.sizeof(_abi.QuantArgs), x_dtype=_abi.F16, x=4096, ldx=256, rows=4, cols=256,
                convrot=0, round_rotated=0, q=8192, ldq=256, scale=16384)
    _expect_invalid('w8a8_quantize_rows', _abi.QuantArgs(**{**base, 'x_dtype': 9}), 'x_dtype')
    _expect_invalid('w8a8_quantize_rows', _abi.QuantArgs(**{**base, 'convrot': 128}), 'convrot')
    _expect_invalid('w8a8_quantize_rows', _abi.QuantArgs(**{**base, 'cols': 24, 'ldx': 24, 'ldq': 24}),
                    'multiple of 16')
    _expect_invalid('w8a8_quantize_rows', _abi.QuantArgs(**{**base, 'x': 4097}), 'aligned')
    _expect_invalid('w8a8_quantize_rows', _abi.QuantArgs(**{**base, 'ldx': 100}), 'leading dimension')
    _expect_invalid('w8a8_quantize_rows', _abi.QuantArgs(**{**base, 'scale': None}), 'go together')
    _expect_invalid('w8a8_quantize_rows', _abi.QuantArgs(**{**base, 'x': None}), 'null x')
    _expect_invalid('w8a8_quantize_rows', _abi.QuantArgs(**{**base, 'q': None, 'scale': None}), 'no output')
    _expect_invalid('w8a8_quantize_rows', _abi.QuantArgs(**{**base, 'row_max': 4096, 'row_max_out': 4096}),
                    'own maximum')
    # ConvRot sign words need the rotation and a 16-byte aligned array
    _expect_invalid('w8a8_quantize_rows', _abi.QuantArgs(**{**base, 'convrot_signs': 4096}), 'convrot_signs')
    _expect_invalid('w8a8_quantize_rows', _abi.QuantArgs(**{**base, 'convrot': 256, 'convrot_signs': 4100}),
                    'convrot_signs')


def test_gemm_argument_checks():
    base = dict(struct_size=ctypes.sizeof(_abi.GemmArgs), epilogue=_abi.EPI_INT32, a=4096, lda=64, b=8192,
                ldb=64, m=16, n=16, k=64, out=16384, ldc=16, out_dtype=_abi.I32)
    _expect_invalid('w8a8_gemm', _abi.GemmArgs(**{**base, 'k': 72, 'lda': 80, 'ldb': 80}), 'multiple of 16')
    _expect_invalid('w8a8_gemm', _abi.GemmArgs(**{**base, 'bias': 4096, 'bias_dtype': _abi.F16}), 'no bias')
    _expect_invalid('w8a8_gemm', _abi.GemmArgs(**{**base, 'out_dtype': _abi.F16}), 'I32')
    _expect_invalid('w8a8_gemm', _abi.GemmArgs(**{**base, 'epilogue': _abi.EPI_ROW, 'out_dtype': _abi.F16}),
                    'row_scale')
    _expect_invalid('w8a8_gemm', _abi.GemmArgs(**{**base, 'epilogue': _abi.EPI_ROW, 'out_dtype': _abi.BF16,
                                                   'row_scale': 64, 'col_scale': 64, 'col_scale_stride': 1,
                                                   'residual': 4096, 'ldr': 16}), 'residual')
    _expect_invalid('w8a8_gemm', _abi.GemmArgs(**{**base, 'k': 1 << 20, 'lda': 1 << 20, 'ldb': 1 << 20}),
                    'overflow')
    _expect_invalid('w8a8_gemm', _abi.GemmArgs(**{**base, 'a': 4100}), 'aligned')


def test_gemm_rope_epilogue_checks():
    lib = _abi.load()
    rope = _abi.RopeEpilogue(heads=2, rot_dim=96, freq_dtype=_abi.F16, eps=1e-6, freqs=4096, q_gain=8192,
                             k_gain=12288)
    base = dict(struct_size=ctypes.sizeof(_abi.GemmArgs), epilogue=_abi.EPI_COLUMN, a=4096, lda=128, b=8192,
                ldb=128, m=256, n=3 * 2 * 128, k=128, row_scale=64, col_scale=128, col_scale_stride=1,
                out=16384, ldc=3 * 2 * 128, out_dtype=_abi.F16)

    def call(rope_fields=None, **gemm_fields):
        r = _abi.RopeEpilogue.from_buffer_copy(rope)
        for key, value in (rope_fields or {}).items():
            setattr(r, key, value)
        args = _abi.GemmArgs(**{**base, **gemm_fields}, rope=ctypes.pointer(r))
        return lib.w8a8_gemm(ctypes.byref(args)), lib.w8a8_last_error().decode()

    rc, msg = call({'heads': 4})
    assert rc == _abi.ERR_INVALID and 'heads' in msg
    rc, msg = call({'rot_dim': 95})
    assert rc == _abi.ERR_INVALID and 'rot_dim' in msg
    rc, msg = call({'freq_dtype': _abi.BF16})
    assert rc == _abi.ERR_INVALID and 'freq_dtype' in msg
    rc, msg = call({'q_gain': 8200})
    assert rc == _abi.ERR_INVALID and 'aligned' in msg
    rc, msg = call({'freq_layout': 2})
    assert rc == _abi.ERR_INVALID and 'freq_layout' in msg
    for rope_fields, gemm_fields in (({'rot_dim': 20}, {}), ({}, {'m': 64}), ({}, {'bias': 64, 'bias_dtype': _abi.F32}),
                                     ({}, {'out_dtype': _abi.F32}), ({}, {'ldc': 3 * 2 * 128 + 4}),
                                     ({}, {'k': 64, 'lda': 64, 'ldb': 64})):
        rc, msg = call(rope_fields, **gemm_fields)
        assert rc == _abi.ERR_UNSUPPORTED and 'rope epilogue' in msg, (rope_fields, gemm_fields, msg)


def test_attention_argument_checks():
    lib = _abi.load()
    assert lib.w8a8_attention_workspace_size(1, 2, 300) == 2 * (2 * 2 + 2) * 128 * 4
    assert lib.w8a8_attention_workspace_size(0, 2, 300) == 0
    base = dict(struct_size=ctypes.sizeof(_abi.AttnPrepareArgs), in_dtype=_abi.F16, q=4096, k=8192, v=12288, b=1,
                h=2, nq=100, nk=300, d=128, sm_scale=0.088, q8=16384, qs=20480, k8=24576, ks=28672, vt8=32768,
                vs=36864, vsum=38912, workspace=40960, workspace_bytes=1 << 20, q_strides=(0, 12800, 128),
                k_strides=(0, 38400, 128), v_strides=(0, 38400, 128))
    _expect_invalid('w8a8_attention_prepare', _abi.AttnPrepareArgs(**{**base, 'd': 64}), 'head dimension')
    _expect_invalid('w8a8_attention_prepare', _abi.AttnPrepareArgs(**{**base, 'in_dtype': _abi.BF16}), 'in_dtype')
    _expect_invalid('w8a8_attention_prepare', _abi.AttnPrepareArgs(**{**base, 'workspace_bytes': 64}), 'workspace')
    _expect_invalid('w8a8_attention_prepare', _abi.AttnPrepareArgs(**{**base, 'k': 8200}), 'aligned')
    _expect_invalid('w8a8_attention_prepare', _abi.AttnPrepareArgs(**{**base, 'sm_scale': 0.0}), 'sm_scale')
    _expect_invalid('w8a8_attention_prepare', _abi.AttnPrepareArgs(**{**base, 'nk': 0}), 'empty')
    _expect_invalid('w8a8_attention_prepare', _abi.AttnPrepareArgs(**{**base, 'k_strides': (0, 38400, 132)}),
                    'multiples of 16 bytes')
    _expect_invalid('w8a8_attention_prepare', _abi.AttnPrepareArgs(**{**base, 'q_strides': (0, -128, 128)}),
                    'multiples of 16 bytes')
    att = dict(struct_size=ctypes.sizeof(_abi.AttentionArgs), out_dtype=_abi.F16, q8=4096, qs=8192, k8=12288,
               ks=16384, vt8=20480, vs=24576, vsum=26624, b=1, h=2, nq=100, nk=300, d=128, sm_scale=0.088,
               out=28672, out_strides=(0, 128, 256))
    _expect_invalid('w8a8_attention', _abi.AttentionArgs(**{**att, 'out_dtype': _abi.I32}), 'out_dtype')
    _expect_invalid('w8a8_attention', _abi.AttentionArgs(**{**att, 'out': None}), 'null')
    _expect_invalid('w8a8_attention', _abi.AttentionArgs(**{**att, 'sm_scale': 0.0}), 'sm_scale')
    _expect_invalid('w8a8_attention', _abi.AttentionArgs(**{**att, 'out_strides': (0, 128, 260)}), '16 bytes')
    # Rows overlap: the heads interleave with a token stride of one row.
    _expect_invalid('w8a8_attention', _abi.AttentionArgs(**{**att, 'out_strides': (0, 128, 128)}), 'overlap')
    _expect_invalid('w8a8_attention', _abi.AttentionArgs(**{**att, 'out_strides': (0, 0, 128)}), 'overlap')
    big = _abi.AttentionArgs(**{**att, 'nk': (1 << 17) + 1})
    assert lib.w8a8_attention(ctypes.byref(big)) == _abi.ERR_UNSUPPORTED
    assert '131072' in lib.w8a8_last_error().decode()


def test_swiglu_argument_checks():
    base = dict(struct_size=ctypes.sizeof(_abi.SwigluArgs), x_dtype=_abi.F16, x=4096, ldx=512, rows=2,
                width=256, q=8192, ldq=256, scale=16384)
    _expect_invalid('w8a8_swiglu_quantize', _abi.SwigluArgs(**{**base, 'width': 320, 'ldx': 640}), 'multiple of 256')
    _expect_invalid('w8a8_swiglu_quantize', _abi.SwigluArgs(**{**base, 'x_dtype': _abi.BF16}), 'x_dtype')
    _expect_invalid('w8a8_swiglu_quantize', _abi.SwigluArgs(**{**base, 'q': None, 'scale': None}), 'no output')
    _expect_invalid('w8a8_swiglu_quantize', _abi.SwigluArgs(**{**base, 'ldx': 256}), 'ldx')
    _expect_invalid('w8a8_swiglu_quantize', _abi.SwigluArgs(**{**base, 'convrot_signs': 4100}), 'convrot_signs')


def test_dequantize_argument_checks():
    base = dict(struct_size=ctypes.sizeof(_abi.DequantArgs), epilogue=_abi.EPI_INT32, acc=4096, ldacc=16, m=4,
                n=16, row_scale=64, col_scale=128, col_scale_stride=1, out=8192, ldc=16, out_dtype=_abi.F16)
    _expect_invalid('w8a8_dequantize', _abi.DequantArgs(**base), 'ROW or COLUMN')
    _expect_invalid('w8a8_dequantize', _abi.DequantArgs(**{**base, 'epilogue': _abi.EPI_ROW,
                                                            'col_scale_stride': 3}), 'stride')


def test_norm_argument_checks():
    base = dict(struct_size=ctypes.sizeof(_abi.NormArgs), x_dtype=_abi.F16, x=4096, ldx=256, rows=4, cols=256,
                eps=1e-6, convrot=256, round_rotated=1, q=8192, ldq=256, q_scale=16384)
    _expect_invalid('w8a8_norm_quantize', _abi.NormArgs(**{**base, 'x_dtype': _abi.F32}), 'x_dtype')
    _expect_invalid('w8a8_norm_quantize', _abi.NormArgs(**{**base, 'q': None}), 'neither y nor q')
    _expect_invalid('w8a8_norm_quantize', _abi.NormArgs(**{**base, 'cols': 272, 'ldx': 272, 'ldq': 272}),
                    'multiple of 256')
    _expect_invalid('w8a8_norm_quantize', _abi.NormArgs(**{**base, 'q_scale': None}), 'q_scale')
    _expect_invalid('w8a8_norm_quantize', _abi.NormArgs(**{**base, 'mod_shift': 4096}), 'together')
    _expect_invalid('w8a8_norm_quantize', _abi.NormArgs(**{**base, 'mod_shift': 4096, 'mod_scale': 8192,
                                                            'ld_mod': 256, 'mod_rows': 3}), 'labels')
    _expect_invalid('w8a8_norm_quantize', _abi.NormArgs(**{**base, 'mod_shift': 4096, 'mod_scale': 8192,
                                                            'ld_mod': 250, 'mod_rows': 3, 'labels': 64}), 'ld_mod')
    _expect_invalid('w8a8_norm_quantize', _abi.NormArgs(**{**base, 'weight': 4100}), 'weight')
    _expect_invalid('w8a8_norm_quantize', _abi.NormArgs(**{**base, 'ldx': 200}), 'ldx')
    _expect_invalid('w8a8_norm_quantize', _abi.NormArgs(**{**base, 'convrot': 0, 'convrot_signs': 4096}),
                    'convrot_signs')
    # without quantization a 16-column multiple is enough
    n = _abi.NormArgs(**{**base, 'q': None, 'q_scale': None, 'y': 8192, 'ldy': 272, 'cols': 272, 'ldx': 272,
                         'rows': 0})
    assert _abi.load().w8a8_norm_quantize(ctypes.byref(n)) == _abi.OK


def test_rms_rope_argument_checks():
    base = dict(struct_size=ctypes.sizeof(_abi.RmsRopeArgs), in_dtype=_abi.F16, packed=4096, ldp=3 * 4 * 128, rows=2,
                heads=4, dim=128, rot_dim=96, freq_dtype=_abi.F16, freqs=8192, q_gain=12288, k_gain=16384,
                eps=1e-6, out_dtype=_abi.F16, q_out=20480, k_out=24576)
    _expect_invalid('w8a8_rms_rope', _abi.RmsRopeArgs(**{**base, 'dim': 64}), 'dim')
    _expect_invalid('w8a8_rms_rope', _abi.RmsRopeArgs(**{**base, 'rot_dim': 95}), 'rot_dim')
    _expect_invalid('w8a8_rms_rope', _abi.RmsRopeArgs(**{**base, 'rot_dim': 130}), 'rot_dim')
    _expect_invalid('w8a8_rms_rope', _abi.RmsRopeArgs(**{**base, 'in_dtype': _abi.BF16}), 'in_dtype')
    _expect_invalid('w8a8_rms_rope', _abi.RmsRopeArgs(**{**base, 'ldp': 4 * 128}), 'ldp')
    _expect_invalid('w8a8_rms_rope', _abi.RmsRopeArgs(**{**base, 'q_out': 20482}), 'aligned')
    _expect_invalid('w8a8_rms_rope', _abi.RmsRopeArgs(**{**base, 'freqs': None}), 'null')
    # 11184816 rows x 24 heads: 6 workgroups of 64 threads per row reach 2^32 work-items
    _expect_invalid('w8a8_rms_rope', _abi.RmsRopeArgs(**{**base, 'rows': 11184816, 'heads': 24,
                                                        'ldp': 2 * 24 * 128}), 'too large')
    n = _abi.RmsRopeArgs(**{**base, 'rows': 0})
    assert _abi.load().w8a8_rms_rope(ctypes.byref(n)) == _abi.OK


def test_empty_problems_return_ok_without_launch():
    lib = _abi.load()
    a = _abi.GemmArgs(struct_size=ctypes.sizeof(_abi.GemmArgs), epilogue=_abi.EPI_INT32, m=0, n=16, k=64,
                      out_dtype=_abi.I32)
    assert lib.w8a8_gemm(ctypes.byref(a)) == _abi.OK
    q = _abi.QuantArgs(struct_size=ctypes.sizeof(_abi.QuantArgs), x_dtype=_abi.F32, rows=0, cols=64)
    assert lib.w8a8_quantize_rows(ctypes.byref(q)) == _abi.OK


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(RuntimeError, match='no CPU fallback'):
        _abi.load(tmp_path / 'libw8a8.so')
