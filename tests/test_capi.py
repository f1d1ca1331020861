"""The C-ABI library: it loads, exports exactly what include/anvil_mi355x.h declares, and reports argument errors
as the exceptions the reference raises. No compute call is made (this file runs without a GPU)."""
import ctypes as C
import re
from pathlib import Path

import pytest

from anvil_mi355x import runtime as rt

HEADER = Path(__file__).resolve().parents[1] / "include" / "anvil_mi355x.h"


def declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(anvil_\w+)\s*\(", text, re.M)))


def test_header_declarations_match_the_binding():
    assert declared() == sorted(rt.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = rt.library()
    for name in declared():
        assert hasattr(lib.cdll, name), name
    assert lib.cdll.anvil_version() == 1


def test_library_leaves_none_of_its_own_symbols_undefined():
    """A kernel whose host launch stub was never emitted shows up as an undefined anvil:: symbol."""
    import subprocess
    out = subprocess.run(["nm", "-D", "--undefined-only", "-C", str(rt.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    assert "anvil" not in out, [l for l in out.splitlines() if "anvil" in l][:5]


def test_null_context_is_a_value_error():
    lib = rt.library()
    with pytest.raises(ValueError, match="null context"):
        lib.call("anvil_sync", None)
    with pytest.raises(ValueError, match="null pointer"):
        lib.call("anvil_gemm_i8", None, None, None, None, 1, 1, 1, 1, 1, None, 1, 0, None, 1)
    with pytest.raises(ValueError):
        lib.call("anvil_init", 0, None)            # null output pointer
    with pytest.raises(ValueError, match="null context"):
        lib.call("anvil_host_alloc", None, 16, None)
    with pytest.raises(ValueError, match="null context"):
        lib.call("anvil_host_free", None, None)
    for name, args in (("anvil_graph_begin", ()), ("anvil_graph_end", (None,)), ("anvil_graph_launch", (None,)),
                       ("anvil_graph_destroy", (None,))):
        with pytest.raises(ValueError, match="null context"):
            lib.call(name, None, *args)


def test_gemm_argument_validation_precedes_the_device():
    """Arguments are validated on the host before any device call (non-null dummies are never dereferenced)."""
    lib = rt.library()
    st = (C.c_int64 * 9)(*[0, 0, 16, 0, 0, 16, 0, 0, 16])
    p = C.c_void_p(4096)
    gemm = lambda *a: lib.call("anvil_gemm_i8_ex", None, p, p, p, *a)   # noqa: E731
    with pytest.raises(ValueError, match="shift 32"):
        gemm(1, 1, 16, 16, 16, st, 1, 32, None, 1, 0)
    with pytest.raises(ValueError, match="non-positive"):
        gemm(1, 1, 0, 16, 16, st, 1, 3, None, 1, 0)
    with pytest.raises(ValueError, match="LUT epilogue needs an i8"):
        gemm(1, 1, 16, 16, 16, st, 1, 3, p, 2, 0)
    with pytest.raises(ValueError, match="SPLITK needs UNCHECKED"):
        gemm(1, 1, 16, 16, 16, st, 1, 3, None, 1, 16)
    with pytest.raises(ValueError, match="SPLITK needs UNCHECKED"):
        gemm(2, 1, 16, 16, 16, st, 1, 3, None, 1, 17)
    with pytest.raises(ValueError, match="unknown flags"):
        gemm(1, 1, 16, 16, 16, st, 1, 3, None, 1, 256)
    with pytest.raises(ValueError, match="K-blocked operands need ANVIL_GEMM_UNCHECKED"):
        gemm(1, 1, 16, 16, 16, st, 1, 3, None, 1, 32)
    with pytest.raises(ValueError, match="K-block stride 16 of Bt out of range"):
        gemm(1, 1, 16, 16, 16, st, 1, 3, None, 1, 1 | 64)
    with pytest.raises(ValueError, match="exclude each other"):
        gemm(1, 1, 16, 16, 16, st, 1, 3, None, 1, 6)
    with pytest.raises(ValueError, match="null context"):
        gemm(1, 1, 16, 16, 16, st, 1, 3, None, 1, 1)


def test_status_codes_map_to_reference_exceptions():
    assert rt._ERRORS == {1: ValueError, 2: OverflowError, 3: ZeroDivisionError, 4: RuntimeError}


def test_no_gpu_here_is_a_runtime_error():
    """anvil_init on a machine without a visible gfx950 device fails loudly (no CPU fallback)."""
    if Path("/dev/kfd").exists():
        pytest.skip("a GPU device node is present")
    out = C.c_void_p()
    with pytest.raises((RuntimeError, ValueError)):
        rt.library().call("anvil_init", 0, C.byref(out))


def test_attention_argument_validation_precedes_the_device():
    lib = rt.library()
    st = (C.c_int64 * 12)(*[64 * 64, 64, 64] * 3 + [64 * 64, 64, 64])
    p = C.c_void_p(4096)
    att = lambda T, D, one, flags, s=st: lib.call("anvil_attention_i8", None, p, p, p, p, 1, 1, T, D, s, 1, 3, p,  # noqa: E731
                                                  one, 1, 1, 3, flags)
    with pytest.raises(ValueError, match="ANVIL_OP_UNCHECKED"):
        att(64, 64, 127, 0)
    with pytest.raises(ValueError, match="multiple of 32"):
        att(48, 64, 127, 1)
    with pytest.raises(ValueError, match="head dim"):
        att(64, 48, 127, 1)
    with pytest.raises(ValueError, match="does not fit int8"):
        att(64, 64, 128, 1)
    bad = (C.c_int64 * 12)(*[64 * 64, 64, 72] + [64 * 64, 64, 64] * 3)
    with pytest.raises(ValueError, match="stride 2"):
        att(64, 64, 127, 1, bad)
    for ldk, ldv in ((32, 64), (64, 48), (1 << 26, 64), (64, 1 << 26)):   # K rows < D apart, V^T rows < T, > 2^31
        s = (C.c_int64 * 12)(*[64 * 64, 64, 64] + [64 * 64, 64, ldk] + [64 * 64, 64, ldv] + [64 * 64, 64, 64])
        with pytest.raises(ValueError, match="K row stride"):
            att(64, 64, 127, 1, s)
    for ldo in (32, 1 << 26):                                       # O rows < D apart, 32 rows past 2^31
        s = (C.c_int64 * 12)(*[64 * 64, 64, 64] * 3 + [64 * 64, 64, ldo])
        with pytest.raises(ValueError, match="O row stride"):
            att(64, 64, 127, 1, s)
    with pytest.raises(ValueError, match="null context"):
        att(64, 64, 127, 1)


def test_rmsnorm_flag_validation_precedes_the_device():
    lib = rt.library()
    p = C.c_void_p(4096)
    rms = lambda flags, cols=768: lib.call("anvil_rmsnorm_int_ex", None, p, 1, p, p, 1024, 1, 14, 0, 0, 4, cols, p,  # noqa: E731
                                           flags)
    with pytest.raises(ValueError, match="unknown flags"):
        rms(8)
    with pytest.raises(ValueError, match="K-blocked result needs cols % 64"):
        rms(rt.OP_UNCHECKED | rt.RMS_OUT_KBLOCK, 80)
    with pytest.raises(ValueError, match="needs ANVIL_OP_UNCHECKED"):
        rms(rt.RMS_S24)
    with pytest.raises(ValueError, match="null context"):
        rms(rt.OP_UNCHECKED | rt.RMS_S24)


def test_gemm_desc_layout_matches_the_header(tmp_path):
    """The ctypes mirror of anvil_gemm_desc has the C struct's size and field offsets (checked with gcc)."""
    import subprocess
    fields = [f for f, _ in rt.GemmDesc._fields_]
    src = tmp_path / "layout.c"
    src.write_text('#include <stddef.h>\n#include <stdio.h>\n#include "anvil_mi355x.h"\nint main(void) {\n'
                   '  printf("%zu", sizeof(anvil_gemm_desc));\n' +
                   "".join(f'  printf(" %zu", offsetof(anvil_gemm_desc, {f}));\n' for f in fields) + "  return 0;\n}\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-I", str(HEADER.parent), str(src), "-o", str(exe)], check=True)
    got = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    assert got == [C.sizeof(rt.GemmDesc)] + [getattr(rt.GemmDesc, f).offset for f in fields]


def test_gemm_group_validates_every_member_first():
    lib = rt.library()
    p = 4096
    good = rt.GemmDesc(A=p, Bt=p, C=p, lut=None, batch0=1, batch1=1, M=16, N=16, K=16, mult=1, shift=3,
                       out_dtype=rt.I8, flags=0)
    good.strides[:] = [0, 0, 16, 0, 0, 16, 0, 0, 16]
    bad = rt.GemmDesc.from_buffer_copy(good)
    bad.shift = 32
    grp = lambda *ds, n=None: lib.call("anvil_gemm_i8_group", None, (rt.GemmDesc * len(ds))(*ds),  # noqa: E731
                                        len(ds) if n is None else n)
    with pytest.raises(ValueError, match="null pointer"):
        lib.call("anvil_gemm_i8_group", None, None, 1)
    with pytest.raises(ValueError, match="count 0"):
        grp(good, n=0)
    with pytest.raises(ValueError, match="count 5"):
        grp(good, good, good, good, good)
    with pytest.raises(ValueError, match="shift 32"):                # the last member fails before any launch
        grp(good, good, bad)
    with pytest.raises(ValueError, match="null context"):
        grp(good, good)
