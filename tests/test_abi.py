"""The C ABI of libhdcmamba_hip.so on the CPU: the library loads, exports every entry
point include/hdcm.h declares, and rejects bad arguments before touching the GPU."""
import ctypes
import re
from pathlib import Path

import pytest
import torch

from hdcmamba_amd import _ops

HEADER = Path(__file__).resolve().parent.parent / "include" / "hdcm.h"
OK, EINVAL, EALIGN, EUNSUPPORTED, ELAUNCH, EWORKSPACE, ETOOBIG = 0, -1, -2, -3, -4, -5, -6


def declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(hdcm_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _ops.lib()
    names = declared()
    assert len(names) >= 9
    for n in names:
        assert hasattr(lib, n), n
    assert sorted(_ops._PROTOS) == names, "ctypes prototypes out of step with include/hdcm.h"


def test_abi_version_and_strerror():
    lib = _ops.lib()
    assert lib.hdcm_abi_version() == _ops.ABI_VERSION
    for code in (OK, EINVAL, EALIGN, EUNSUPPORTED, ELAUNCH, EWORKSPACE):
        assert lib.hdcm_strerror(code)
    assert b"unknown" in lib.hdcm_strerror(123)


def test_workspace_sizes():
    lib = _ops.lib()
    # header + (A, H) words of 16 bytes per channel and 512-row tile
    assert lib.hdcm_ssm_workspace_bytes(1, 32768, 128) == 2048 + 128 * 64 * 16
    assert lib.hdcm_ssm_workspace_bytes(0, 10, 4) == 0
    n = lib.hdcm_slot_workspace_bytes(1, 32768, 1024, 16, 64, _ops.HDCM_BF16)
    assert n > 0 and n % (2 * 16 * 64 * 64 * 4) == 0
    assert lib.hdcm_slot_workspace_bytes(1, 64, 200, 5, 64, _ops.HDCM_BF16) == 0  # head dim 40
    assert lib.hdcm_slot_workspace_bytes(1, 64, 576, 4, 64, _ops.HDCM_BF16) == 0  # head dim 144
    assert lib.hdcm_slot_workspace_bytes(1, 64, 240, 5, 64, _ops.HDCM_BF16) > 0   # head dim 48
    assert lib.hdcm_slot_workspace_bytes(1, 96, 256, 4, 48, _ops.HDCM_BF16) > 0   # chunk 48
    assert lib.hdcm_slot_workspace_bytes(1, 100, 256, 4, 48, _ops.HDCM_BF16) == 0  # L not a multiple of C


P16 = ctypes.c_void_p(16 * 1024)       # aligned non-null stand-ins: never dereferenced,
P17 = ctypes.c_void_p(16 * 1024 + 2)   # every call below fails validation first
P20 = ctypes.c_void_p(16 * 1024 + 4)   # 4-byte aligned only
P24 = ctypes.c_void_p(16 * 1024 + 8)   # 8-byte aligned only


def test_norm_conv_validation():
    f = _ops.lib().hdcm_norm_conv_fwd
    args = [P16, 256 * 64, 64, P16, P16, P16, P16, P16, 256 * 64, 64, 1, 256, 64, 1e-5, 1, None]
    bad_null = list(args); bad_null[0] = None
    assert f(*bad_null) == EINVAL
    bad_align = list(args); bad_align[0] = P17
    assert f(*bad_align) == EALIGN
    bad_d = list(args); bad_d[12] = 63
    assert f(*bad_d) == EALIGN
    bad_dtype = list(args); bad_dtype[14] = 7
    assert f(*bad_dtype) == EUNSUPPORTED
    empty = list(args); empty[11] = 0
    assert f(*empty) == OK  # nothing to do, no launch


def test_ssm_validation():
    f = _ops.lib().hdcm_ssm_fwd
    base = [P16, 3 * 64 + 8, P16, None, P16, 64, None, None, 0, P16, 1 << 20, 1, 256, 64, 1, None]
    a = list(base); a[9] = None
    assert f(*a) == EWORKSPACE
    a = list(base); a[10] = 16
    assert f(*a) == EWORKSPACE
    a = list(base); a[1] = 100
    assert f(*a) == EINVAL
    a = list(base); a[0] = P17
    assert f(*a) == EALIGN
    # row statistics: a part stride of at least B*L pairs, 8-byte aligned
    a = list(base); a[7], a[8] = P16, 255
    assert f(*a) == EINVAL
    a = list(base); a[7], a[8] = P20, 256
    assert f(*a) == EALIGN


def test_ssm_noalloc_validation():
    """The no-allocation scan checks like hdcm_ssm_fwd and rejects inputs whose scratch would
    exceed its fixed array before any HIP call."""
    f = _ops.lib().hdcm_ssm_fwd_noalloc
    base = [P16, 3 * 64 + 8, P16, None, P16, 64, None, None, 0, 1, 256, 64, 1, None]
    a = list(base); a[1] = 100
    assert f(*a) == EINVAL
    a = list(base); a[0] = P17
    assert f(*a) == EALIGN
    a = list(base); a[9] = 0
    assert f(*a) == OK  # empty: nothing to do
    a = list(base); a[9], a[10], a[11] = 64, 32768, 128  # 48 MiB of scratch
    a[1], a[5] = 3 * 128, 128
    assert f(*a) == ETOOBIG
    assert b"scratch" in _ops.lib().hdcm_strerror(ETOOBIG)


def test_slot_validation():
    lib = _ops.lib()
    st = lib.hdcm_slot_state_fwd
    base = [P16, 3 * 64 + 4 * 256, 3 * 64, P16, None, P16, 1 << 24, 1, 256, 256, 4, 64, 1, None]
    a = list(base); a[10] = 5  # 256 % 5 != 0
    assert st(*a) == EINVAL
    a = list(base); a[8] = 250  # L not a multiple of C
    assert st(*a) == EINVAL
    a = list(base); a[9] = 200; a[10] = 5; a[1] = 3 * 64 + 4 * 200  # head dim 40: not a multiple of 16
    assert st(*a) == EUNSUPPORTED
    a = list(base); a[5] = None
    assert st(*a) == EWORKSPACE
    a = list(base); a[1] = 256  # row too short for q,k,v,gate
    assert st(*a) == EINVAL
    g = lib.hdcm_slot_gate_fwd
    gb = [P16, 3 * 64 + 4 * 256, 3 * 64, P16, P16, P16, 1e-5, P16, 1 << 24, P16, 64 + 256, 64, None,
          None, 0, 1, 256, 256, 4, 64, 1, None]
    a = list(gb); a[11] = 62  # output runs of 4 must stay aligned
    assert g(*a) == EALIGN
    a = list(gb); a[10] = 200  # output row too short
    assert g(*a) == EINVAL
    a = list(gb); a[13], a[14] = P16, 255  # row statistics need a part stride of B*L pairs
    assert g(*a) == EINVAL
    a = list(gb); a[13], a[14] = P20, 256
    assert g(*a) == EALIGN


def test_decode_step_validation():
    lib = _ops.lib()
    # hdcm_norm_conv_step_fwd(x, x_rs, ln_w, ln_b, conv_w, conv_b, hist, out, out_rs, B, D, eps, dtype, stream)
    f = lib.hdcm_norm_conv_step_fwd
    base = [P16, 256, P16, P16, P16, P16, P16, P16, 256, 4, 256, 1e-5, 1, None]
    a = list(base); a[6] = None  # no history buffer
    assert f(*a) == EINVAL
    a = list(base); a[10] = 250  # D not whole 16-byte groups
    a[1] = a[8] = 250
    assert f(*a) == EALIGN
    a = list(base); a[10] = a[1] = a[8] = 8 * 4 * 256 + 8  # wider than the kernel's row tiling
    assert f(*a) == EUNSUPPORTED
    a = list(base); a[9] = 0
    assert f(*a) == OK
    # hdcm_mixer_step_fwd(projs, prs, q_col, A_log, h, gamma, S_prev, S_intra, pos, C, gn_w, gn_b, eps,
    #                     out, ors, y_col, g_col, B, dm, ds, H, dtype, stream)
    g = lib.hdcm_mixer_step_fwd
    P = 3 * 64 + 4 * 256
    gb = [P16, P, 3 * 64, P16, P16, P16, P16, P16, 0, None, 64, P16, P16, 1e-5, P16, 64 + 256, 0, 64, 4, 256,
          64, 4, 1, None]
    a = list(gb); a[8] = 64  # pos must be inside the chunk
    assert g(*a) == EINVAL
    a = list(gb); a[7] = None  # S_intra
    assert g(*a) == EINVAL
    a = list(gb); a[19] = 1040; a[21] = 4; a[1] = 3 * 64 + 4 * 1040  # head dim 260
    a[15] = 64 + 1040
    assert g(*a) == EUNSUPPORTED
    a = list(gb); a[15] = 200  # output row too short
    assert g(*a) == EINVAL
    a = list(gb); a[18] = 0
    assert g(*a) == OK
    assert lib.hdcm_chunk_pos_advance(None, 64, None) == EINVAL


def test_gnorm_gate_validation():
    # hdcm_gnorm_gate_fwd(y1, y1_rs, y2, y2_rs, gate, g_rs, gn_w, gn_b, eps, out, o_rs, row_stats, sps, rows,
    #                     dm, H, dtype, stream)
    f = _ops.lib().hdcm_gnorm_gate_fwd
    base = [P16, 512, P16, 512, P16, 2048, P16, P16, 1e-5, P16, 640, None, 0, 4, 512, 2, 1, None]
    a = list(base); a[16] = 2  # unknown dtype
    assert f(*a) == EUNSUPPORTED
    a = list(base); a[0] = None
    assert f(*a) == EINVAL
    a = list(base); a[15] = 3  # d_model not a multiple of the heads
    assert f(*a) == EINVAL
    a = list(base); a[14] = 1024; a[15] = 1; a[1] = a[3] = a[5] = a[10] = 1024  # head dim 1024
    assert f(*a) == EUNSUPPORTED
    a = list(base); a[14] = 510; a[15] = 2  # odd head dim with a second part
    assert f(*a) == EUNSUPPORTED
    a = list(base); a[11] = P16; a[12] = 3  # statistics part stride below the row count
    assert f(*a) == EINVAL
    a = list(base); a[13] = 0
    assert f(*a) == OK


def test_skinny_gemm_validation():
    # hdcm_skinny_gemm_fwd(A, a_rs, W, w_rs, bias, res, res_rs, out, o_rs, M, N, K, dtype, stream)
    f = _ops.lib().hdcm_skinny_gemm_fwd
    base = [P16, 2048, P16, 2048, None, None, 0, P16, 8576, 16, 8576, 2048, 1, None]
    a = list(base); a[12] = 0  # fp32 is not built (decode in fp32 stays on the library GEMM)
    assert f(*a) == EUNSUPPORTED
    a = list(base); a[9] = 17  # more than 16 rows
    assert f(*a) == EUNSUPPORTED
    a = list(base); a[11] = 2040; a[1] = a[3] = 2040  # K not a multiple of 32
    assert f(*a) == EUNSUPPORTED
    a = list(base); a[11] = 4096; a[1] = a[3] = 4096  # K beyond the per-wave register share
    assert f(*a) == EUNSUPPORTED
    a = list(base); a[2] = None
    assert f(*a) == EINVAL
    a = list(base); a[8] = 100  # output row shorter than N
    assert f(*a) == EINVAL
    a = list(base); a[1] = 2052; a[3] = 2052  # rows not 16-byte aligned
    assert f(*a) == EALIGN
    a = list(base); a[9] = 0
    assert f(*a) == OK


def test_launch_options_round_trip():
    """Every option the Python wrapper names exists in the library, keeps a value it is set to,
    rejects values out of range and unknown options (no GPU involved)."""
    lib = _ops.lib()
    for name, key in _ops.OPTIONS.items():
        old = lib.hdcm_get_option(key)
        assert lib.hdcm_set_option(key, 1) == OK, name
        assert lib.hdcm_get_option(key) == 1, name
        assert lib.hdcm_set_option(key, -1) == EINVAL, name
        assert lib.hdcm_set_option(key, old) == OK, name
    assert lib.hdcm_set_option(max(_ops.OPTIONS.values()) + 1, 0) == EINVAL
    assert lib.hdcm_set_option(0, 0) == EINVAL
    assert lib.hdcm_get_option(99) == 0
    assert lib.hdcm_set_option(_ops.OPTIONS["skinny_fold_tail"], 2) == EINVAL


def test_norm_conv_in_proj_step_validation():
    # hdcm_norm_conv_in_proj_step_fwd(x, x_rs, ln_w, ln_b, conv_w, conv_b, hist, eps, u, u_rs, W, w_rs, bias,
    #                                 out, o_rs, B, D, N, ws, ws_bytes, dtype, stream)
    lib = _ops.lib()
    f = lib.hdcm_norm_conv_in_proj_step_fwd
    wsb = lib.hdcm_step_workspace_bytes()
    assert wsb >= 128 * 19  # the tag, the timeouts, 8 flag copies, 9 counters: a 128-byte line each
    base = [P16, 2048, P16, P16, P16, P16, P16, 1e-5, P16, 2048, P16, 2048, None, P16, 8576, 16, 2048, 8576,
            P16, wsb, 1, None]
    a = list(base); a[20] = 0  # fp32 is not built
    assert f(*a) == EUNSUPPORTED
    a = list(base); a[15] = 17  # more than 16 rows
    assert f(*a) == EUNSUPPORTED
    a = list(base); a[15] = 0
    assert f(*a) == EINVAL
    a = list(base); a[16] = 2080; a[1] = a[9] = a[11] = 2080  # d_model beyond 2048
    assert f(*a) == EUNSUPPORTED
    a = list(base); a[16] = 2040; a[1] = a[9] = a[11] = 2040  # not a multiple of 32
    assert f(*a) == EUNSUPPORTED
    a = list(base); a[18] = None
    assert f(*a) == EWORKSPACE
    a = list(base); a[19] = wsb - 4
    assert f(*a) == EWORKSPACE
    a = list(base); a[6] = None  # no history
    assert f(*a) == EINVAL
    a = list(base); a[14] = 100  # output row shorter than N
    assert f(*a) == EINVAL
    a = list(base); a[9] = 2052  # u rows not 16-byte aligned
    assert f(*a) == EALIGN
    a = list(base); a[18] = ctypes.c_void_p(16 * 1024 + 64)  # workspace not on a 128-byte line
    assert f(*a) == EALIGN


def test_gemm_validation():
    # hdcm_gemm_fwd(x, x_rs, w, w_rs, bias, out, o_rs, M, N, K, dtype, stream)
    f = _ops.lib().hdcm_gemm_fwd
    base = [P16, 1024, P16, 1024, None, P16, 4480, 300, 4480, 1024, 1, None]
    a = list(base); a[10] = 0  # fp32 is not built
    assert f(*a) == EUNSUPPORTED
    a = list(base); a[0] = None
    assert f(*a) == EINVAL
    a = list(base); a[6] = 100  # output row shorter than N
    assert f(*a) == EINVAL
    a = list(base); a[9] = 1020; a[1] = a[3] = 1020  # K not a multiple of 8
    assert f(*a) == EALIGN
    a = list(base); a[8] = 4478; a[6] = 4478  # N not a multiple of 4
    assert f(*a) == EALIGN
    a = list(base); a[1] = 1 << 22  # row stride beyond 32-bit tile offsets
    assert f(*a) == EUNSUPPORTED
    a = list(base); a[7] = 0; a[0] = a[5] = None  # no rows
    assert f(*a) == OK
    # hdcm_rowln_gemm_fwd(c, c_rs, w, w_rs, res, r_rs, out, o_rs, M, N, K, eps, dtype, stream)
    h = _ops.lib().hdcm_rowln_gemm_fwd
    base = [P16, 1152, P16, 1152, P16, 1024, P16, 1024, 300, 1024, 1152, 1e-5, 1, None]
    a = list(base); a[4] = None  # no residual
    assert h(*a) == EINVAL
    a = list(base); a[5] = 100  # residual row shorter than N
    assert h(*a) == EINVAL
    a = list(base); a[12] = 0
    assert h(*a) == EUNSUPPORTED
    a = list(base); a[8] = 0; a[0] = a[4] = a[6] = None
    assert h(*a) == OK
    # hdcm_rowln_gemm_stats_fwd(c, c_rs, w, w_rs, w_sums, row_stats, parts, part_stride, res, r_rs, out,
    #                           o_rs, M, N, K, eps, dtype, stream)
    g = _ops.lib().hdcm_rowln_gemm_stats_fwd
    base = [P16, 1152, P16, 1152, P16, P16, 18, 300, P16, 1024, P16, 1024, 300, 1024, 1152, 1e-5, 1, None]
    a = list(base); a[5] = None  # no row statistics
    assert g(*a) == EINVAL
    a = list(base); a[4] = None  # no weight sums
    assert g(*a) == EINVAL
    a = list(base); a[6] = 0
    assert g(*a) == EINVAL
    a = list(base); a[7] = 299  # part stride shorter than the rows
    assert g(*a) == EINVAL
    a = list(base); a[13] = 1020; a[9] = a[11] = 1020  # 16-byte output runs need N % 8 == 0
    assert g(*a) == EALIGN
    a = list(base); a[8] = P24  # residual not 16-byte aligned
    assert g(*a) == EALIGN
    a = list(base); a[16] = 0
    assert g(*a) == EUNSUPPORTED
    a = list(base); a[12] = 0; a[0] = a[8] = a[10] = None
    assert g(*a) == OK
    # hdcm_row_sums_fwd(w, w_rs, N, K, sums, dtype, stream)
    r = _ops.lib().hdcm_row_sums_fwd
    assert r(P16, 1152, 1024, 1152, None, 1, None) == EINVAL
    assert r(P16, 1152, 1024, 1150, P16, 1, None) == EALIGN
    assert r(P16, 1152, 1024, 1152, P16, 0, None) == EUNSUPPORTED
    assert r(None, 1152, 0, 1152, None, 1, None) == OK


def test_norm_conv_bwd_validation():
    lib = _ops.lib()
    assert lib.hdcm_norm_conv_bwd_workspace_bytes(1, 32768, 1024) == 32768 * 8 + 512 * 7 * 1024 * 4  # 64-row chunks
    assert lib.hdcm_norm_conv_bwd_workspace_bytes(0, 10, 64) == 0
    # hdcm_norm_conv_bwd(go, g_bs, g_rs, x, x_bs, x_rs, ln_w, ln_b, conv_w, dx, d_bs, d_rs,
    #                    d_ln_w, d_ln_b, d_conv_w, d_conv_b, ws, ws_bytes, B, L, D, eps, dtype, stream)
    f = lib.hdcm_norm_conv_bwd
    ws_n = lib.hdcm_norm_conv_bwd_workspace_bytes(2, 64, 256)
    base = [P16, 64 * 256, 256, P16, 64 * 256, 256, P16, P16, P16, P16, 64 * 256, 256,
            P16, P16, P16, P16, P16, ws_n, 2, 64, 256, 1e-5, 1, None]
    a = list(base); a[12] = None  # no d_ln_w
    assert f(*a) == EINVAL
    a = list(base); a[17] = ws_n - 1  # short workspace
    assert f(*a) == EWORKSPACE
    a = list(base); a[20] = 8192; a[2] = a[5] = a[11] = 8192; a[1] = a[4] = a[10] = 64 * 8192  # D too wide
    assert f(*a) == EUNSUPPORTED
    a = list(base); a[20] = 250; a[2] = a[5] = a[11] = 250; a[1] = a[4] = a[10] = 64 * 250
    assert f(*a) == EALIGN
    # B == 0 zeroes the parameter gradients on the GPU (tests/test_gpu_block.py covers it)


def test_rowln_validation():
    f = _ops.lib().hdcm_rowln_fwd
    base = [P16, 1152, P16, 1152, None, None, 10, 1152, 1e-5, 1, None]
    a = list(base); a[4] = P16  # w without b
    assert f(*a) == EINVAL
    a = list(base); a[7] = 1150
    assert f(*a) == EALIGN
    a = list(base); a[7] = 8 * 13 * 64  # wider than the kernel's register tiling
    a[1] = a[3] = a[7]
    assert f(*a) == EUNSUPPORTED


def test_rowln_bwd_validation():
    lib = _ops.lib()
    assert lib.hdcm_rowln_bwd_workspace_bytes(32768, 1024) == 1024 * 2 * 1024 * 4  # 1024 workgroups at most
    assert lib.hdcm_rowln_bwd_workspace_bytes(10, 1024) == 3 * 2 * 1024 * 4       # ceil(10 / 4)
    assert lib.hdcm_rowln_bwd_workspace_bytes(-1, 1024) == 0
    # hdcm_rowln_bwd(dy, dy_rs, x, x_rs, w, dx, dx_rs, dw, db, ws, ws_bytes, rows, width, eps, dtype, stream)
    f = lib.hdcm_rowln_bwd
    ws_n = lib.hdcm_rowln_bwd_workspace_bytes(10, 1024)
    base = [P16, 1024, P16, 1024, P16, P16, 1024, P16, P16, P16, ws_n, 10, 1024, 1e-5, 1, None]
    a = list(base); a[7] = None  # affine without dw
    assert f(*a) == EINVAL
    a = list(base); a[10] = ws_n - 1  # short workspace
    assert f(*a) == EWORKSPACE
    a = list(base); a[4] = a[7] = a[8] = a[9] = None; a[10] = 0  # no affine: no workspace needed
    a[11] = 0
    assert f(*a) == OK
    a = list(base); a[12] = 1020; a[1] = a[3] = a[6] = 1020  # rows not whole 16-byte groups
    assert f(*a) == EALIGN
    a = list(base); a[12] = 8 * 9 * 64; a[1] = a[3] = a[6] = a[12]  # wider than the backward's tiling
    assert f(*a) == EUNSUPPORTED
    a = list(base); a[0] = None  # null input with rows to process
    assert f(*a) == EINVAL
    a = list(base); a[14] = 2
    assert f(*a) == EUNSUPPORTED


def test_backward_entry_points_validation():
    lib = _ops.lib()
    # hdcm_slot_attend_fwd(base, rs, q_col, k_col, v_col, gamma, phi, ws, ws_bytes, out, ors, out_col,
    #                      chain, chain_rs, B, L, dm, H, C, dtype, stream)
    f = lib.hdcm_slot_attend_fwd
    ws_n = lib.hdcm_slot_workspace_bytes(1, 128, 256, 4, 64, 1)
    base = [P16, 1024, 256, 512, 0, P16, 0, P16, ws_n, P16, 256, 0, None, 0, 1, 128, 256, 4, 64, 1, None]
    a = list(base); a[1] = 700  # row shorter than the v block at column 512 + 256
    assert f(*a) == EINVAL
    a = list(base); a[3] = 516  # block not on a 16-byte boundary
    assert f(*a) == EALIGN
    a = list(base); a[1] = -1024; a[10] = -256; a[15] = 0  # negative strides accepted (empty: no launch)
    assert f(*a) == OK
    a = list(base); a[8] = ws_n - 1
    assert f(*a) == EWORKSPACE
    a = list(base); a[16] = 200; a[17] = 5  # head dim 40: not a multiple of 16
    assert f(*a) == EUNSUPPORTED
    a = list(base); a[12] = P16; a[13] = 200  # chain rows shorter than out's block
    assert f(*a) == EINVAL
    a = list(base); a[12] = P16; a[13] = 258  # chain rows not 8-byte aligned
    assert f(*a) == EALIGN
    # hdcm_ssm_bwd(projs, prs, A_log, h, hrs, gy, gyrs, dprojs, drs, dA, ws, ws_bytes, B, L, ds, dtype, stream)
    g = lib.hdcm_ssm_bwd
    n = lib.hdcm_ssm_bwd_workspace_bytes(1, 100, 64, 1)
    assert n > 0 and lib.hdcm_ssm_bwd_workspace_bytes(0, 100, 64, 1) == 0
    gb = [P16, 192, P16, P16, 64, P16, 64, P16, 192, P16, P16, n, 1, 100, 64, 1, None]
    a = list(gb); a[9] = None  # no d A_log
    assert g(*a) == EINVAL
    a = list(gb); a[11] = n - 1
    assert g(*a) == EWORKSPACE
    a = list(gb); a[8] = 100  # dprojs rows shorter than 3*ds
    assert g(*a) == EINVAL
    # hdcm_gnorm_gate_bwd(y, yrs, gate, grs, gn_w, gn_b, eps, dout, dors, dy, dyrs, dgate, dgrs, dgn_w, dgn_b,
    #                     ws, ws_bytes, rows, dm, H, dtype, stream)
    h = lib.hdcm_gnorm_gate_bwd
    m = lib.hdcm_gnorm_gate_bwd_workspace_bytes(256, 4)
    assert m == max(4 * 256 * 2 * 64 * 4, 512 * 2 * 256 * 4)  # per-head form, row-stripe form
    hb = [P16, 256, P16, 256, P16, P16, 1e-5, P16, 256, P16, 256, P16, 256, P16, P16, P16, m, 10, 256, 4, 1, None]
    a = list(hb); a[19] = 5  # dm not a multiple of H
    assert h(*a) == EINVAL
    a = list(hb); a[18] = 200; a[19] = 5  # head dim 40: not a multiple of 16
    assert h(*a) == EUNSUPPORTED
    a = list(hb); a[16] = m - 1
    assert h(*a) == EWORKSPACE
    # hdcm_slot_phi_prep / hdcm_slot_phi_chain(projs, prs, q_col, z|dprojs, rs, rows, dm, dtype, stream)
    assert lib.hdcm_slot_phi_prep(P16, 1024, 192, P16, 800, 10, 256, 1, None) == EINVAL  # z rows < 4*dm
    assert lib.hdcm_slot_phi_prep(P16, 1224, 196, P16, 1024, 10, 256, 1, None) == EALIGN
    assert lib.hdcm_slot_phi_chain(P16, 600, 192, P16, 1216, 10, 256, 1, None) == EINVAL  # projs rows short
    assert lib.hdcm_slot_phi_chain(None, 1216, 192, None, 1216, 0, 256, 1, None) == OK


def test_cpu_tensors_raise():
    """No CPU fallback: the product path refuses host tensors."""
    from hdcmamba_amd import HdcMamba9v3Block, HdcMamba9v3Model

    blk = HdcMamba9v3Block(64, 16, 2, 64)
    with pytest.raises(RuntimeError, match="GPU"):
        blk(torch.randn(1, 64, 64))
    with pytest.raises(RuntimeError, match="GPU"):
        HdcMamba9v3Model(64, 1, 16, 32, 2)(torch.randn(1, 64, 64))
    with pytest.raises(RuntimeError, match="GPU"):
        _ops.norm_conv(torch.randn(1, 4, 64), torch.ones(64), torch.zeros(64), torch.zeros(64, 4),
                       torch.zeros(64), 1e-5)
