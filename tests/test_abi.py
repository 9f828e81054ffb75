"""The C-ABI library: it loads, exports every symbol include/*.h declares,
and its host-side logic (kernel table, config enumeration, argument
rejection) behaves like the reference's -- all without touching a GPU."""
import ctypes
import os
import re
import subprocess
import sys

import pytest

import bmb

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h)
           for h in ("kernels.h", "gemm.h", "flash.h", "attention.h", "nn.h", "gpt.h")]


def _declared():
    names = set()
    for h in HEADERS:
        src = open(h).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        src = re.sub(r"^#pragma.*$", "", src, flags=re.M)
        for m in re.finditer(r"\b([A-Za-z_]\w*)\s*\(", src):
            name = m.group(1)
            if name in ("if", "sizeof", "defined", "sgemm_fn", "void") or name.startswith("BMB_"):
                continue
            names.add(name)
        # the C++ view's inline overloads are not exported symbols
        names.discard("return")
        for m in re.finditer(r"extern\s+const\s+\w+\s+(\w+)", src):
            names.add(m.group(1))
        for m in re.finditer(r"extern\s+const\s+char\s*\*\s*const\s+(\w+)", src):
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


def test_exports_nothing_undeclared():
    """The library's dynamic symbol table is the C ABI of include/*.h: no C++
    symbol (kernel host stubs, internal helpers, standard-library template
    instantiations) is visible to a program that links it. The __hip_cuid_*
    markers are the HIP compiler's per-source identifiers."""
    rows = [l.split() for l in os.popen("nm -D --defined-only %s" % bmb.LIB_PATH).read().splitlines()]
    names = {r[-1] for r in rows if len(r) >= 3}
    extra = sorted(n for n in names - _declared() if not n.startswith("__hip_cuid_"))
    assert not extra, extra


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


def test_gpt_struct_layout_matches_header(tmp_path):
    """The ctypes mirror of struct GPT has the C header's size and offsets
    (compiled with the host C compiler; no GPU)."""
    import subprocess
    fields = [f[0] for f in bmb.GPT._fields_]
    src = ["#include <stdio.h>", "#include <stddef.h>", '#include "gpt.h"', "int main(void){",
           'printf("%zu\\n", sizeof(GPT));']
    src += ['printf("%%zu\\n", offsetof(GPT, %s));' % f for f in fields]
    src += ['printf("%%zu\\n", offsetof(Activations, %s));' % f for f in bmb.ACT_NAMES]
    src += ['printf("%%zu\\n", offsetof(Gradients, %s));' % f for f in bmb.GRAD_ACT_NAMES]
    src += ["return 0;}"]
    c = tmp_path / "layout.c"
    c.write_text("\n".join(src))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-I", os.path.join(ROOT, "include"), str(c), "-o",
                    str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True,
                                          check=True).stdout.split()]
    want = [ctypes.sizeof(bmb.GPT)] + [getattr(bmb.GPT, f).offset for f in fields]
    want += [getattr(bmb.Activations, f).offset for f in bmb.ACT_NAMES]
    want += [getattr(bmb.Gradients, f).offset for f in bmb.GRAD_ACT_NAMES]
    assert got == want


def test_gpt_param_sizes_and_names():
    """param_sizes is host code: compare with the oracle's src/gpt.cu:32-50
    restatement at the GPT-2 small config and the gradient-check config."""
    import oracle as O
    for cfg in ((1024, 50257, 50304, 12, 12, 768), (64, 65, 128, 2, 4, 128)):
        assert bmb.param_sizes(cfg) == O.gpt_param_sizes(cfg)
    assert sum(bmb.param_sizes((1024, 50257, 50304, 12, 12, 768))) == 124475904
    assert bmb.param_names() == list(bmb.PARAM_NAMES) == list(O.PARAM_NAMES)


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus N > 1 exits with status 2 and says
    why, before it touches the GPU or imports torch."""
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""
