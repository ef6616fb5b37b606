"""CPU-side checks of the C-ABI library: it loads, exports every symbol the
public header declares, its RNG equals the oracle's, and the structs the
Python binding passes match the header layout. No GPU work is launched."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from lumen_amd import _native
from oracle import oracle as o

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    src = open(os.path.join(ROOT, "include", "lumen_sampler.h")).read()
    return sorted(set(re.findall(r"^\s*(?:int|void|float|uint64_t|uint32_t|const char \*)\s*\*?\s*"
                                 r"(lumen_\w+)\s*\(", src, re.M)))


def test_library_exports_every_header_symbol():
    L = _native.load()
    names = header_functions()
    assert len(names) >= 8
    for n in names:
        assert hasattr(L, n), n
    assert set(names) == set(_native.EXPORTS)
    out = subprocess.run(["nm", "-D", "--defined-only", _native.LIB_PATH], capture_output=True,
                         text=True).stdout
    exported = set(re.findall(r" T (lumen_\w+)", out))
    assert set(names) <= exported


def test_library_embeds_code_object():
    out = subprocess.run(["nm", "-D", "--defined-only", _native.LIB_PATH], capture_output=True,
                         text=True).stdout
    assert "lumen_gfx950_code_object" in out
    hsaco = os.path.join(os.path.dirname(_native.LIB_PATH), "lumen_sampler_gfx950.hsaco")
    assert os.path.getsize(hsaco) > 10_000
    assert open(hsaco, "rb").read(4) == b"\x7fELF"


def test_version_string():
    assert b"gfx950" in _native.load().lumen_sampler_version()


def test_rng_matches_oracle():
    L = _native.load()
    for seed in (0, 1, 42, 12345, 0xC0FFEE, 2**64 - 1):
        a = ctypes.c_uint64(L.lumen_xorshift64_new(seed))
        b = o.Xorshift64(seed)
        assert a.value == b.state.value
        for _ in range(50):
            assert L.lumen_xorshift64_next_f32(ctypes.byref(a)) == b.next_f32()


def test_python_mirror_rng_and_params():
    from lumen_amd.sampling import SamplingParams, Xorshift64

    r = Xorshift64(42)
    assert 0.0 < r.next_f32() < 1.0
    assert SamplingParams(repetition_penalty=1.0).penalties_active() is False
    assert SamplingParams(repetition_penalty=1.0 + 1e-8).penalties_active() is False
    assert SamplingParams(repetition_penalty=1.05).penalties_active() is True
    assert SamplingParams(presence_penalty=0.5).penalties_active() is True


def test_params_validate_wire_ranges():
    # crates/lumen-server/src/wire/openai.rs:357-381: the closed ranges
    # [0, 2] and [0, 1] with both ends accepted; NaN, infinities and any
    # value just outside rejected, with the field named in the message
    from lumen_amd.sampling import SamplingParams

    f32 = np.float32
    ok_t = [0.0, 1e-30, 1.0, 2.0, float(np.nextafter(f32(2.0), f32(0.0)))]
    bad_t = [float("nan"), float("inf"), -float("inf"), -1e-30,
             float(np.nextafter(f32(2.0), f32(3.0))), 2.5, -1.0]
    ok_p = [None, 0.0, 0.5, 1.0]
    bad_p = [float("nan"), float("inf"), -1e-30, float(np.nextafter(f32(1.0), f32(2.0))), 1.5]
    for t in ok_t:
        for q in ok_p:
            SamplingParams(temperature=t, top_p=q).validate()
    for t in bad_t:
        with pytest.raises(ValueError, match="temperature must be between 0 and 2"):
            SamplingParams(temperature=t).validate()
    for q in bad_p:
        with pytest.raises(ValueError, match="top_p must be between 0 and 1"):
            SamplingParams(temperature=1.0, top_p=q).validate()
    # temperature is checked first, as in the reference
    with pytest.raises(ValueError, match="temperature"):
        SamplingParams(temperature=3.0, top_p=3.0).validate()
    L = _native.load()
    assert L.lumen_sampling_params_validate(None) != 0


def test_struct_layouts():
    # lumen_sampling_params: 6 floats, 2 u64, 2 i32 = 48 bytes
    assert ctypes.sizeof(_native.SamplingParamsC) == 48
    assert ctypes.sizeof(_native.RowTraceC) == 64
    assert ctypes.sizeof(_native.BatchC) == 176
    assert ctypes.sizeof(_native.TokenBytesC) == 24


def test_struct_layouts_match_the_header(tmp_path):
    # every field offset of the ctypes mirrors equals the C compiler's
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    structs = {"lumen_batch": _native.BatchC, "lumen_sampling_params": _native.SamplingParamsC,
               "lumen_row_trace": _native.RowTraceC, "lumen_token_bytes": _native.TokenBytesC}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "lumen_sampler.h"',
             "int main(void) {"]
    want = []
    for cname, py in structs.items():
        lines.append(f'printf("%zu\\n", sizeof({cname}));')
        want.append(ctypes.sizeof(py))
        for f in py._fields_:
            lines.append(f'printf("%zu\\n", offsetof({cname}, {f[0]}));')
            want.append(getattr(py, f[0]).offset)
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(root, "include"), "-o", str(exe), str(src)],
                   check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True,
                                          check=True).stdout.split()]
    assert got == want


def test_create_without_gpu_fails_cleanly():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    L = _native.load()
    h = ctypes.c_void_p()
    rc = L.lumen_sampler_create(ctypes.byref(h), 0)
    assert rc in (_native.LUMEN_ERR_NO_DEVICE, _native.LUMEN_ERR_HIP)
    assert not h.value


def test_device_expf_table_is_exp2():
    src = open(os.path.join(ROOT, "lumen_amd", "csrc", "expf_glibc.h")).read()
    vals = [int(x, 16) for x in re.findall(r"0x([0-9a-f]{16})ull", src)]
    assert vals == o.expf_table()


def test_device_expf_constants_match_oracle():
    # the polynomial and shift constants of the device restatement are the
    # ones the oracle's CPU twin uses (and that twin equals libm's expf)
    dev = open(os.path.join(ROOT, "lumen_amd", "csrc", "expf_glibc.h")).read()
    cpu = open(os.path.join(ROOT, "oracle", "glibc_expf.c")).read()
    for c in ("0x1.c6af84b912394p-5", "0x1.ebfce50fac4f3p-3", "0x1.62e42ff0c52d6p-1",
              "0x1.8p+52", "0x1.71547652b82fep+0", "0x1.62e42ep6f", "0x1.9fe368p6f"):
        assert c in dev and c in cpu, c


def test_code_object_exports_abi_stamp():
    # The library refuses a code object whose kernel-argument layout stamp
    # differs from its own (sampler_host.cpp, lumen_sampler_create); the
    # stamp is the exported symbol lumen_kernel_abi.
    hsaco = os.path.join(ROOT, "lumen_amd", "lib", "lumen_sampler_gfx950.hsaco")
    readelf = "/opt/rocm/llvm/bin/llvm-readelf"
    if not (os.path.exists(hsaco) and os.path.exists(readelf)):
        pytest.skip("code object or llvm-readelf not present")
    out = subprocess.run([readelf, "--symbols", hsaco], capture_output=True, text=True).stdout
    line = [l for l in out.splitlines() if l.split() and l.split()[-1] == "lumen_kernel_abi"]
    assert line and "OBJECT" in line[0]
