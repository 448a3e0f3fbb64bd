"""Properties of the built gfx950 code (no GPU needed).

Every kernel of libvqk_hip.so must run without scratch (private-segment) memory.  A
scratch frame - an outlined device function, or an array the compiler could not keep in
registers - changes no result, so the parity tests cannot see it, but it made the lm_head
kernels 14-22 us slower per call.  The check reads the AMDGPU code-object metadata of the
library's own device code: the `.hip_fatbin` section holds one offload bundle per
translation unit, and each bundle's gfx950 entry is an ELF whose notes list every
kernel's `.private_segment_fixed_size`.
"""
import os
import shutil
import struct
import subprocess

import pytest

LIB = os.path.join(os.path.dirname(__file__), "..", "vllm-quant-kernels_amd", "vllm_quant_kernels",
                   "libvqk_hip.so")
READELF = "/opt/rocm/llvm/bin/llvm-readelf"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def _gfx950_code_objects(fatbin: bytes):
    """Yield the gfx950 code objects of every offload bundle in a .hip_fatbin section
    (bundle layout: magic, u64 entry count, then per entry u64 offset, u64 size, u64 triple
    length and the triple; offsets are relative to the bundle start)."""
    p = fatbin.find(MAGIC)
    while p != -1:
        n = struct.unpack_from("<Q", fatbin, p + len(MAGIC))[0]
        q = p + len(MAGIC) + 8
        for _ in range(n):
            off, size, tl = struct.unpack_from("<QQQ", fatbin, q)
            q += 24
            triple = fatbin[q:q + tl].decode()
            q += tl
            if "gfx950" in triple and size:
                yield fatbin[p + off:p + off + size]
        p = fatbin.find(MAGIC, p + 1)


def _kernel_private_bytes(tmp_path):
    fb = tmp_path / "fatbin.bin"
    subprocess.run(["objcopy", f"--dump-section=.hip_fatbin={fb}", LIB, str(tmp_path / "lib.o")],
                   check=True, capture_output=True)
    out = {}
    for i, co in enumerate(_gfx950_code_objects(fb.read_bytes())):
        path = tmp_path / f"co{i}.o"
        path.write_bytes(co)
        notes = subprocess.run([READELF, "--notes", str(path)], check=True, capture_output=True,
                               text=True).stdout
        name = None
        for line in notes.splitlines():
            t = line.strip()
            if t.startswith(".name:"):
                name = t.split(":", 1)[1].strip()
            elif t.startswith(".private_segment_fixed_size:") and name is not None:
                out[name] = int(t.split(":", 1)[1])
                name = None
    return out


@pytest.mark.skipif(not os.path.exists(LIB), reason="libvqk_hip.so not built")
@pytest.mark.skipif(not (os.path.exists(READELF) and shutil.which("objcopy")),
                    reason="ROCm llvm-readelf or objcopy missing")
def test_no_kernel_uses_scratch(tmp_path):
    sizes = _kernel_private_bytes(tmp_path)
    assert any("lmhead_lds_kernel" in k for k in sizes), "no lm_head kernels found in the library"
    assert any("gumbel_surv_kernel" in k for k in sizes)
    with_scratch = {k: v for k, v in sizes.items() if v != 0}
    assert not with_scratch, with_scratch
