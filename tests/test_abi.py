"""The C ABI library loads, exports every declared symbol, and rejects bad
arguments on the host before any GPU work (CPU only)."""

import ctypes
import re
from pathlib import Path

import pytest

from qvex import _C

REPO = Path(__file__).resolve().parent.parent


def declared_symbols():
    names = []
    for h in sorted((REPO / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names += re.findall(r"\b(qvex_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_header_declares_symbols():
    assert "qvex_qmv_w4g64" in declared_symbols()


def test_library_exports_every_declared_symbol():
    lib = _C.lib()
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert not missing, f"libqvex.so lacks {missing}"


def test_bindings_cover_header():
    assert set(declared_symbols()) <= set(_C.exported_symbols())


def test_abi_version():
    assert _C.lib().qvex_abi_version() == _C.ABI_VERSION


@pytest.mark.parametrize("M,N,K", [(0, 16, 64), (9, 16, 64), (1, 0, 64), (1, 16, 96), (1, 16, 0)])
def test_qmv_rejects_bad_shapes(M, N, K):
    buf = ctypes.create_string_buffer(1 << 16)
    p = ctypes.addressof(buf)
    p16 = (p + 15) // 16 * 16
    with pytest.raises(_C.QvexError, match="qvex_qmv_w4g64"):
        _C.call("qvex_qmv_w4g64", p16, p16, p16, p16, p16, M, N, K, None)


def test_qmv_rejects_misaligned_pointer():
    buf = ctypes.create_string_buffer(1 << 12)
    p16 = (ctypes.addressof(buf) + 15) // 16 * 16
    with pytest.raises(_C.QvexError, match="16-byte"):
        _C.call("qvex_qmv_w4g64", p16 + 2, p16, p16, p16, p16, 1, 16, 64, None)


def test_qmv_rejects_unknown_tile():
    buf = ctypes.create_string_buffer(1 << 12)
    p16 = (ctypes.addressof(buf) + 15) // 16 * 16
    with pytest.raises(_C.QvexError, match="tile"):
        _C.call("qvex_qmv_w4g64_tiled", p16, p16, p16, p16, p16, 1, 16, 64, 3, 1, None)


@pytest.mark.parametrize("kps,D,err", [(64, 256, "multiple of 128"), (192, 256, "multiple of 128"),
                                       (128, 64, "128 or 256")])
def test_attention_rejects_bad_split_or_dim(kps, D, err):
    buf = ctypes.create_string_buffer(1 << 12)
    p16 = (ctypes.addressof(buf) + 15) // 16 * 16
    with pytest.raises(_C.QvexError, match=err):
        _C.call("qvex_attention", p16, p16, p16, p16, 4, 16, 4, D, 4096, 4096, 4096, kps, p16, 2 * D * 16, p16, p16,
                1 << 40, None)


def test_packed_bytes_and_rejections():
    lib = _C.lib()
    assert lib.qvex_w4g64_packed_bytes(16, 256) == 2304
    assert lib.qvex_w4g64_packed_bytes(17, 512) == 2 * 2 * 2304
    assert lib.qvex_w4g64_packed_bytes(16, 320) == 0
    assert lib.qvex_w4g64_packed_bytes(0, 256) == 0
    buf = ctypes.create_string_buffer(1 << 12)
    p16 = (ctypes.addressof(buf) + 15) // 16 * 16
    with pytest.raises(_C.QvexError, match="outside 1..8"):
        _C.call("qvex_qmv_w4g64_packed", p16, p16, p16, 9, 16, 256, None)
    with pytest.raises(_C.QvexError, match="multiple of 256"):
        _C.call("qvex_qmv_w4g64_packed", p16, p16, p16, 1, 16, 320, None)
    with pytest.raises(_C.QvexError, match="unsupported tile"):
        _C.call("qvex_qmv_w4g64_packed_tiled", p16, p16, p16, 1, 16, 256, 3, 1, -1, None)
    with pytest.raises(_C.QvexError, match="packed buffer"):
        _C.call("qvex_w4g64_pack", p16, p16, p16, 16, 256, p16, 2303, None)


def test_packed_swiglu_rejects_odd_halves():
    buf = ctypes.create_string_buffer(1 << 16)
    p16 = (ctypes.addressof(buf) + 15) // 16 * 16
    with pytest.raises(_C.QvexError, match="multiple of 16"):
        _C.call("qvex_qmv_w4g64_packed_swiglu", p16, p16, p16, 1, 24, 256, None)
    with pytest.raises(_C.QvexError, match="multiple of 16"):
        _C.call("qvex_w4g64_pack_swiglu", p16, p16, p16, 24, 256, p16, 1 << 15, None)


def test_spec_filter_argument_rules():
    buf = ctypes.create_string_buffer(1 << 20)
    p16 = (ctypes.addressof(buf) + 15) // 16 * 16
    with pytest.raises(_C.QvexError, match="top_k"):
        _C.call("qvex_spec_accept_filtered", p16, None, p16, p16, p16, 1.0, None, 0.0, -1, 0.9, p16, p16,
                1, 1, 4096, p16, 1 << 19, None)
    with pytest.raises(_C.QvexError, match="top_p is NaN"):
        _C.call("qvex_spec_accept_filtered", p16, None, p16, p16, p16, 1.0, None, 0.0, 0, float("nan"), p16, p16,
                1, 1, 4096, p16, 1 << 19, None)
    with pytest.raises(_C.QvexError, match="workspace"):       # the wide form needs its row records
        _C.call("qvex_spec_accept_filtered", p16, None, p16, p16, p16, 1.0, None, 0.0, 0, 0.9, p16, p16,
                1, 1, 4096, p16, 8, None)
    lib = _C.lib()
    assert lib.qvex_spec_accept_filtered_workspace_bytes(1, 1, 8192, 0, 20) > \
        lib.qvex_spec_accept_filtered_workspace_bytes(1, 1, 8192, 0, 0) == lib.qvex_spec_accept_workspace_bytes(1, 1, 8192, 0)


def test_gdn_decode_fused_argument_rules():
    buf = ctypes.create_string_buffer(1 << 12)
    p = (ctypes.addressof(buf) + 15) // 16 * 16
    C, kd = 2 * 256 + 512, 256

    def call(T=4, Hk=2, Hv=4, Dk=128, Dv=128, conv_dim=C, key_dim=kd, R=67, n_slots=9, stride=C + 512 + 8):
        _C.call("qvex_gdn_decode_fused", p, stride, p, R, p, p, 4, conv_dim, key_dim, 1.0, 1.0, 1e-6, p, p, C,
                C + 512, p, n_slots, 1, p, 1e-6, p, T, Hk, Hv, Dk, Dv, None)

    with pytest.raises(_C.QvexError, match="1..8"):
        call(T=9)
    with pytest.raises(_C.QvexError, match="Dk = Dv = 128"):
        call(Dk=64)
    with pytest.raises(_C.QvexError, match="multiple of Hk"):
        call(Hk=3)
    with pytest.raises(_C.QvexError, match="do not match"):
        call(conv_dim=C + 128)
    with pytest.raises(_C.QvexError, match="ring_rows"):
        call(R=6)
    with pytest.raises(_C.QvexError, match="n_slots"):
        call(n_slots=4)
    with pytest.raises(_C.QvexError, match="projection row"):
        call(stride=C + 100)


def test_gdn_decode_split_argument_rules():
    buf = ctypes.create_string_buffer(1 << 12)
    p = (ctypes.addressof(buf) + 15) // 16 * 16
    C, kd = 2 * 256 + 512, 256

    def call(T=4, nb=8, Dk=128, n_slots=9, R=67):
        _C.call("qvex_gdn_decode_split", p, C + 512 + 8, p, R, p, p, 4, C, kd, 1.0, 1.0, 1e-6, p, p, C, C + 512,
                p, n_slots, 1, p, p, p, T, 2, 4, Dk, 128, nb, None)

    for nb in (0, 1, 3, 16):
        with pytest.raises(_C.QvexError, match="blocks_per_head"):
            call(nb=nb)
    with pytest.raises(_C.QvexError, match="1..8"):
        call(T=9)
    with pytest.raises(_C.QvexError, match="Dk = Dv = 128"):
        call(Dk=64)
    with pytest.raises(_C.QvexError, match="n_slots"):
        call(n_slots=4)
    with pytest.raises(_C.QvexError, match="ring_rows"):
        call(R=6)
    with pytest.raises(_C.QvexError, match="null pointer"):
        _C.call("qvex_gdn_decode_split", p, C + 520, p, 67, p, p, 4, C, kd, 1.0, 1.0, 1e-6, p, p, C, C + 512,
                p, 9, 1, p, p, None, 4, 2, 4, 128, 128, 8, None)


def test_gnorm_resid_argument_rules():
    buf = ctypes.create_string_buffer(1 << 14)
    p = (ctypes.addressof(buf) + 15) // 16 * 16
    for nb in (0, 3, 16):
        with pytest.raises(_C.QvexError, match="seg_nb"):
            _C.call("qvex_qmv_w4g64_packed_gnorm_resid", p, p, 1, 16, 256, p, nb, 1e-6, p, p, p, p, p, None)
    with pytest.raises(_C.QvexError, match="null pointer"):
        _C.call("qvex_qmv_w4g64_packed_gnorm_resid", p, p, 1, 16, 256, None, 8, 1e-6, p, p, p, p, p, None)
    with pytest.raises(_C.QvexError, match="outside 1..8"):
        _C.call("qvex_qmv_w4g64_packed_gnorm_resid", p, p, 9, 16, 256, p, 8, 1e-6, p, p, p, p, p, None)


def test_resid_norm_products_argument_rules():
    buf = ctypes.create_string_buffer(1 << 14)
    p = (ctypes.addressof(buf) + 15) // 16 * 16
    with pytest.raises(_C.QvexError, match="null pointer"):
        _C.call("qvex_qmv_w4g64_packed_resid", p, p, 1, 16, 256, None, p, p, p, p, None)
    with pytest.raises(_C.QvexError, match="outside 1..8"):
        _C.call("qvex_qmv_w4g64_packed_resid", p, p, 9, 16, 256, p, p, p, p, p, None)
    with pytest.raises(_C.QvexError, match="ceil\\(dim/16\\)"):
        _C.call("qvex_qmv_w4g64_packed_rstd", p, p, p, 1, 16, 256, p, 255, 4096, 1e-6, 0, None)
    with pytest.raises(_C.QvexError, match="ceil\\(dim/16\\)"):
        _C.call("qvex_qmv_w4g64_packed_rstd", p, p, p, 1, 16, 256, p, 320, 5120, 1e-6, 0, None)
    with pytest.raises(_C.QvexError, match="16-byte"):
        _C.call("qvex_qmv_w4g64_packed_rstd", p, p, p, 1, 16, 256, p + 4, 256, 4096, 1e-6, 0, None)


def test_dequant_argument_rules():
    buf = ctypes.create_string_buffer(1 << 12)
    p = (ctypes.addressof(buf) + 15) // 16 * 16
    with pytest.raises(_C.QvexError, match="multiple of 64"):
        _C.call("qvex_w4g64_dequant", p, p, p, 4, 96, p, None)
    with pytest.raises(_C.QvexError, match="null pointer"):
        _C.call("qvex_w4g64_dequant", p, None, p, 4, 64, p, None)
    with pytest.raises(_C.QvexError, match="16-byte"):
        _C.call("qvex_w4g64_dequant", p, p, p, 4, 64, p + 2, None)
