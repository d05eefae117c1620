"""The C-ABI library loads, exports what include/sps_attn.h declares, and validates arguments
before touching the GPU. The validation calls pass fake device addresses, so they run only where no
GPU is visible: a call whose arguments passed validation could otherwise launch a kernel on them."""

import ctypes as C
import re
from pathlib import Path

import pytest

from sps_amd import _native as N

HEADER = Path(__file__).resolve().parents[1] / "include" / "sps_attn.h"


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sps_[a-z0-9_]+)\s*\(", text)))


def test_header_declarations_match_binding():
    assert _declared_functions() == sorted(N.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = N.lib()
    for name in _declared_functions():
        assert hasattr(lib, name), name
    assert lib.sps_version().startswith(b"sps_attn")


def _no_gpu() -> bool:
    import torch

    return not torch.cuda.is_available()


cpu_only = pytest.mark.skipif(not _no_gpu(), reason="fake device addresses: CPU build only")


def _fwd(**over):
    args = dict(family=1, B=1, H=1, N=64, D=64, dtype=N.DTYPE_BF16, sm_scale=0.125, window=4, has_pkw=0, pkw=-1,
                docs=None, docs_dtype=N.DTYPE_I64, ws=None, ws_bytes=0, ptr=0x10000, strides=(64 * 64, 64 * 64, 64))
    args.update(over)
    st = N.i64_array(args["strides"])
    p = args["ptr"]
    lse = 0x20000
    return N.lib().sps_attn_fwd(
        args["family"], args["B"], args["H"], args["N"], args["D"], args["dtype"],
        p, st, p, st, p, st, p, st, lse, args["docs"], args["docs_dtype"], 0,
        args["sm_scale"], args["window"], args["has_pkw"], args["pkw"], args["ws"], args["ws_bytes"], None,
    )


@pytest.mark.parametrize(
    "over,code,needle",
    [
        (dict(family=7), N.SPS_E_INVALID, "family"),
        (dict(N=63), N.SPS_E_INVALID, "even"),
        (dict(D=512), N.SPS_E_UNSUPPORTED, "head_dim"),
        (dict(D=48), N.SPS_E_UNSUPPORTED, "head_dim"),
        (dict(dtype=N.DTYPE_F32), N.SPS_E_UNSUPPORTED, "dtype"),
        (dict(ptr=0x10008), N.SPS_E_INVALID, "aligned"),
        (dict(strides=(64 * 64, 64 * 64, 60)), N.SPS_E_INVALID, "multiple of 8"),
        (dict(docs=0x30000, docs_dtype=N.DTYPE_F32), N.SPS_E_INVALID, "int32 or int64"),
        (dict(docs=0x30000, docs_dtype=N.DTYPE_I64, ws_bytes=0), N.SPS_E_WORKSPACE, "workspace"),
        # any finite scale is taken (zero and negative ones included); NaN and infinities are not
        (dict(sm_scale=float("nan")), N.SPS_E_INVALID, "sm_scale"),
        (dict(sm_scale=float("inf")), N.SPS_E_INVALID, "sm_scale"),
        (dict(sm_scale=float("-inf")), N.SPS_E_INVALID, "sm_scale"),
    ],
)
@cpu_only
def test_forward_argument_validation(over, code, needle):
    assert _fwd(**over) == code
    assert needle in N.last_error()


@cpu_only
def test_empty_problem_is_a_noop():
    assert _fwd(B=0) == N.SPS_OK
    assert _fwd(N=0) == N.SPS_OK


def test_workspace_sizes():
    lib = N.lib()
    assert lib.sps_attn_workspace_bytes(1, 4, 16, 4096, 0, 0) == 0
    with_docs = lib.sps_attn_workspace_bytes(1, 4, 16, 4096, 1, 0)
    assert with_docs >= 2 * 4 * (4096 // 32) * 8
    bwd = lib.sps_attn_workspace_bytes(1, 4, 16, 4096, 1, 1)
    assert bwd >= with_docs + 4 * 16 * 4096 * 4
    scans = N.i64_array([64, 4096])
    dec = lib.sps_decode_workspace_bytes(64, 16, 64, 1, N.DTYPE_BF16, 2, scans)
    # D = 64 bf16: 512-key chunks (4 waves x 8 rows x 16 passes) -> 1 + 8 chunks of (64 + 4) floats.
    assert dec >= 64 * 16 * (1 + 8) * (64 + 4) * 4


def _decode(nq=1, D=64, n_seg=0, q_dtype=N.DTYPE_BF16, extra_dtype=N.DTYPE_BF16, n_extra=0):
    z = N.i64_array([0, 0, 0])
    return N.lib().sps_decode(1, 1, D, nq, 0x1000, q_dtype, z, N.DTYPE_BF16, n_seg, None, z, None, z, None, None,
                              None, z, n_extra, None, None, extra_dtype, z, None, 0.125, 0x2000, z, None, 0, None)


@cpu_only
def test_decode_argument_validation():
    assert _decode(nq=3) == N.SPS_E_INVALID and "nq" in N.last_error()
    assert _decode(D=48) == N.SPS_E_UNSUPPORTED
    assert _decode(n_seg=4) == N.SPS_E_INVALID and "segments" in N.last_error()
    assert _decode(q_dtype=N.DTYPE_I32) == N.SPS_E_UNSUPPORTED and "query dtype" in N.last_error()
    assert _decode(n_extra=1, extra_dtype=N.DTYPE_I64) == N.SPS_E_UNSUPPORTED and "extra" in N.last_error()


def test_last_error_truncates():
    _fwd(family=9)
    buf = C.create_string_buffer(8)
    full = N.lib().sps_last_error(buf, len(buf))
    assert full > 7 and len(buf.value) == 7


def test_cached_stride_arrays():
    a = N.i64_const((3, 5, 7))
    assert list(a) == [3, 5, 7] and N.i64_const((3, 5, 7)) is a
    assert list(N.i64_const((3, 5, 8))) == [3, 5, 8]
    for i in range(1100):  # past the cache bound: emptied and refilled, values still right
        assert N.i64_const((i, -i))[1] == -i
    assert list(N.i64_const((3, 5, 7))) == [3, 5, 7]


@cpu_only
def test_backward_pass_selector_validation():
    lib = N.lib()
    st = N.i64_array((64 * 64, 64 * 64, 64))
    p = 0x10000
    for bad in (0, 4, 8, 16 | 1):
        rc = lib.sps_attn_bwd_pass(bad, 1, 1, 1, 64, 64, N.DTYPE_BF16, p, st, p, st, p, st, p, st, p, st, 0x20000,
                                   p, st, p, st, p, st, None, N.DTYPE_I64, 0, 0.125, 4, 0, -1, None, 0, None)
        assert rc == N.SPS_E_INVALID, bad
        assert "pass selector" in N.last_error()
    for bad_scale in (float("nan"), float("inf")):
        rc = lib.sps_attn_bwd_pass(N.BWD_DQ | N.BWD_DKDV, 1, 1, 1, 64, 64, N.DTYPE_BF16, p, st, p, st, p, st, p, st,
                                   p, st, 0x20000, p, st, p, st, p, st, None, N.DTYPE_I64, 0, bad_scale, 4, 0, -1,
                                   0x50000, 0x40000, None)
        assert rc == N.SPS_E_INVALID and "sm_scale" in N.last_error()


def _kv_update(window=2, ring_storage=4, kv_dtype=N.DTYPE_BF16, new_dtype=N.DTYPE_BF16, len_dtype=N.DTYPE_I64,
               active_dtype=N.DTYPE_U8, ret_k=0x3000, B=1):
    z = N.i64_array([0] * 8)
    p = 0x1000
    return N.lib().sps_kv_update(B, 1, 64, kv_dtype, p, p, z, ring_storage, window, p, p, z, ret_k, p, z, 8, p, z,
                                 len_dtype, new_dtype, p, p, p, p, z, p, active_dtype, 1, None)


@cpu_only
def test_kv_update_argument_validation():
    assert _kv_update(window=5, ring_storage=4) == N.SPS_E_INVALID and "ring storage" in N.last_error()
    assert _kv_update(kv_dtype=N.DTYPE_I32) == N.SPS_E_UNSUPPORTED and "cache dtype" in N.last_error()
    assert _kv_update(new_dtype=N.DTYPE_I64) == N.SPS_E_UNSUPPORTED and "new K/V" in N.last_error()
    assert _kv_update(len_dtype=N.DTYPE_F32) == N.SPS_E_INVALID and "lengths" in N.last_error()
    assert _kv_update(active_dtype=N.DTYPE_BF16) == N.SPS_E_INVALID and "active mask" in N.last_error()
    assert _kv_update(ret_k=None) == N.SPS_E_INVALID and "null pointer" in N.last_error()
    assert _kv_update(B=0) == N.SPS_OK


def _rope(D=64, in_dtype=N.DTYPE_F32, ptr=0x10000, st=(4096, 64, 64)):
    s = N.i64_array(st)
    f = N.i64_array((0, 32))
    return N.lib().sps_rope_qkv(1, 1, 1, D, in_dtype, ptr, s, ptr, s, None, None, 0x20000, f, N.DTYPE_BF16,
                                0x30000, s, 0x30000, s, None, None, None)


@cpu_only
def test_rope_argument_validation():
    assert _rope(D=12) == N.SPS_E_UNSUPPORTED and "multiple of 8" in N.last_error()
    assert _rope(in_dtype=N.DTYPE_I32) == N.SPS_E_UNSUPPORTED and "input dtype" in N.last_error()
    assert _rope(ptr=0x10004) == N.SPS_E_INVALID and "aligned" in N.last_error()
    assert _rope(st=(4096, 66, 64)) == N.SPS_E_INVALID and "aligned" in N.last_error()


def _decode_kv_update(len_dtype=N.DTYPE_I64, nq=1, window=2, ring_storage=4, ws_bytes=1 << 20):
    z = N.i64_array([0] * 8)
    p = 0x1000
    return N.lib().sps_decode_kv_update(
        1, 1, 64, nq, 0x1000, N.DTYPE_BF16, z, N.DTYPE_BF16, 0, None, z, None, z, None, None, None, z, 0, None, None,
        N.DTYPE_BF16, z, None, 0.125, 0x2000, z,
        p, p, z, ring_storage, window, p, p, z, p, p, z, 8, p, z, len_dtype, N.DTYPE_BF16, p, p, p, p, z, p,
        N.DTYPE_U8, 1, 0x50000, ws_bytes, None)


@cpu_only
def test_decode_kv_update_argument_validation():
    # The update's arguments are checked before the decode's, and nothing is launched on failure.
    assert _decode_kv_update(len_dtype=N.DTYPE_F32) == N.SPS_E_INVALID and "lengths" in N.last_error()
    assert _decode_kv_update(window=5) == N.SPS_E_INVALID and "ring storage" in N.last_error()
    assert _decode_kv_update(nq=3) == N.SPS_E_INVALID and "nq" in N.last_error()
    scans = N.i64_array([64, 4096])
    lib = N.lib()
    assert lib.sps_decode_kv_update_workspace_bytes(64, 16, 64, 1, N.DTYPE_BF16, 2, scans) >= \
        lib.sps_decode_workspace_bytes(64, 16, 64, 1, N.DTYPE_BF16, 2, scans) + 64 * 16 * 8 * 8
