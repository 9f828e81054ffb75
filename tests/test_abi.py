"""The C-ABI library: it loads, exports every symbol include/*.h declares,
and its host-side logic (kernel table, config enumeration, argument
rejection) behaves like the reference's -- all without touching a GPU."""
import ctypes
import os
import re

import pytest

import bmb

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("kernels.h", "gemm.h", "flash.h")]


def _declared():
    names = set()
    for h in HEADERS:
        src = open(h).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        for m in re.finditer(r"\b([A-Za-z_]\w*)\s*\(", src):
            name = m.group(1)
            if name in ("if", "sizeof", "defined", "sgemm_fn", "void") or name.startswith("BMB_"):
                continue
            names.add(name)
        for m in re.finditer(r"extern\s+const\s+\w+\s+(\w+)", src):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol():
    L = bmb.lib()
    declared = _declared()
    assert {"gemm", "batched_gemm", "flash_attention_forward", "find_kernel",
            "KERNELS", "NUM_KERNELS", "sgemm_doublebuffer"} <= declared
    missing = [n for n in sorted(declared) if not hasattr(L, n)]
    assert not missing, missing
    # and the binding knows the signature of each one
    assert declared <= set(bmb.exported_symbols())


def test_exports_are_c_linkage():
    out = os.popen("nm -D --defined-only %s" % bmb.LIB_PATH).read().split()
    for n in _declared():
        assert n in out, "%s not exported with C linkage" % n


def test_kernel_table():
    table = bmb.kernels()
    assert [t[0] for t in table] == list(range(1, 11))
    names = [t[1] for t in table]
    # ids 1-9 keep the reference's names (src/registry.cu:5-13)
    assert names[:9] == ["naive", "coalesced", "smem", "tile1d", "tile2d", "vectorized",
                         "warptile", "dbuffer", "tensorcore"]
    assert all(0 < t[3] <= 1e-4 for t in table)
    assert bmb.find_kernel(8)["name"] == "dbuffer"
    assert bmb.find_kernel(0) is None and bmb.find_kernel(42) is None


def test_flash_config_enumeration():
    fw, bw = bmb.flash_configs(), bmb.flash_bwd_configs()
    assert len(fw) >= 1 and len(bw) >= 1
    assert 0 <= bmb.flash_default_config() < len(fw)
    assert 0 <= bmb.flash_default_bwd_config() < len(bw)
    L = bmb.lib()
    assert L.flash_config_name(-1) == b"?" and L.flash_config_name(len(fw)) == b"?"
    assert L.flash_bwd_config_name(len(bw)) == b"?"


@pytest.mark.parametrize("C,NH", [(96, 2), (768, 7), (64, 0), (100, 3)])
def test_flash_cfg_rejects_unsupported_heads(C, NH):
    """src/flash.cu:407-412: hs outside {32, 64, 128} -> false, nothing launched
    (rejected on the host, so this runs without a GPU)."""
    p = ctypes.c_void_p(16)
    for cfg in range(len(bmb.flash_configs())):
        assert not bmb.flash_forward_cfg(cfg, p, p, p, 2, 8, C, NH)
    for cfg in range(len(bmb.flash_bwd_configs())):
        assert not bmb.flash_backward_cfg(cfg, p, p, p, p, p, p, 2, 8, C, NH)


def test_flash_cfg_rejects_unknown_ids():
    p = ctypes.c_void_p(16)
    assert not bmb.flash_forward_cfg(-1, p, p, p, 2, 8, 128, 2)
    assert not bmb.flash_forward_cfg(len(bmb.flash_configs()), p, p, p, 2, 8, 128, 2)
    assert not bmb.flash_backward_cfg(99, p, p, p, p, p, p, 2, 8, 128, 2)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(bmb, "_lib", None)
    monkeypatch.setattr(bmb, "LIB_PATH", str(tmp_path / "nope.so"))
    with pytest.raises(RuntimeError):
        bmb.lib()
