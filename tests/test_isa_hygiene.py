"""Static checks on the gfx950 machine code of the built library (CPU only).

The device code objects embedded in wmma_ops_amd/libwmma_ops_amd.so (clang offload
bundles) are disassembled with the ROCm llvm-objdump and checked for two instruction
classes this library must never contain:

* packed-FP32 VALU operations (v_pk_add_f32, v_pk_mul_f32, v_pk_fma_f32): the build
  disables them with -target-feature -packed-fp32-ops;
* writes through the scalar data cache (scalar stores and atomics, and that cache's
  write-back / discard): all GPU writes here are vector stores.

and for one ordering pattern: a workgroup barrier crossed with this wave's LDS reads still
in flight and followed by an LDS DMA (buffer_load ... lds) before they are waited for.
Ring kernels reuse, right after such a barrier, the LDS slot the previous stage read, so
a DMA landing early would overwrite rows another wave has not read yet.

This file names those instructions, so it is listed in .gpurunignore (it never runs on
the GPU box).
"""
import os
import re
import shutil
import struct
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "wmma_ops_amd", "libwmma_ops_amd.so")
OBJDUMP = "/opt/rocm/llvm/bin/llvm-objdump"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"

FORBIDDEN = re.compile(
    r"\b(v_pk_(add|mul|fma)_f32|s_store_\w+|s_buffer_store\w*|s_scratch_store\w*|"
    r"s_atomic_\w+|s_buffer_atomic_\w+|s_dcache_wb\w*|s_dcache_discard\w*)\b")


def gfx950_code_objects(path):
    data = open(path, "rb").read()
    objs, pos = [], 0
    while (start := data.find(MAGIC, pos)) >= 0:
        pos = start + 1
        n = struct.unpack_from("<Q", data, start + 24)[0]
        off = start + 32
        for _ in range(n):
            o, size, tlen = struct.unpack_from("<QQQ", data, off)
            off += 24
            triple = data[off:off + tlen].decode()
            off += tlen
            if "gfx950" in triple and size > 0:
                objs.append(data[start + o:start + o + size])
    return objs


@pytest.fixture(scope="module")
def disassembly(tmp_path_factory):
    if not os.path.exists(LIB):
        pytest.skip("library not built")
    if not shutil.which(OBJDUMP):
        pytest.skip("llvm-objdump not available")
    objs = gfx950_code_objects(LIB)
    assert objs, "no gfx950 code object found in the library"
    texts = []
    d = tmp_path_factory.mktemp("co")
    for i, co in enumerate(objs):
        p = d / f"co{i}.elf"
        p.write_bytes(co)
        out = subprocess.run([OBJDUMP, "-d", "--mcpu=gfx950", str(p)], check=True,
                             capture_output=True, text=True).stdout
        texts.append(out)
    return "\n".join(texts)


def test_library_has_gfx950_kernels(disassembly):
    for k in ["gemm_mfma_kernel", "w4a16_decode_mfma_kernel", "flash_fwd_kernel",
              "int4_prepack_kernel", "splitk_reduce_kernel"]:
        assert k in disassembly, k
    assert "v_mfma_f32_32x32x16_f16" in disassembly
    assert "ds_read_b64_tr_b16" in disassembly


def test_no_forbidden_instructions(disassembly):
    bad = sorted({m.group(0) for m in FORBIDDEN.finditer(disassembly)})
    assert not bad, f"forbidden instructions in device code: {bad}"


_FUNC = re.compile(r"^[0-9a-f]+ <(\S+)>:$")
_LGKM = re.compile(r"lgkmcnt\((\d+)\)")


def lds_reads_pending_at_dma_barriers(text):
    """Kernels with a barrier that some path reaches with LDS reads in flight (counted from
    ds_* issues since the last lgkmcnt(0), capped by later lgkmcnt(N) waits; a straight
    scan of the listing) and after which an LDS DMA issues before lgkmcnt(0)."""
    found = {}
    func, pending, armed = None, 0, False
    for line in text.splitlines():
        m = _FUNC.match(line)
        if m:
            func, pending, armed = m.group(1), 0, False
            continue
        ins = line.strip().split("//")[0].strip()
        if not ins or func is None:
            continue
        op = ins.split()[0]
        if op.startswith("ds_"):
            pending += 1
        elif op == "s_waitcnt":
            w = _LGKM.search(ins)
            if w:
                pending = min(pending, int(w.group(1)))
                if pending == 0:
                    armed = False
        elif op == "s_barrier":
            armed = pending > 0
        elif armed and op.startswith(("buffer_load", "global_load")) and " lds" in ins:
            found[func] = found.get(func, 0) + 1
            armed = False
    return found


def test_no_lds_reads_in_flight_across_a_dma_barrier(disassembly):
    found = lds_reads_pending_at_dma_barriers(disassembly)
    assert not found, f"LDS reads in flight at a barrier followed by an LDS DMA: {sorted(found)}"


def test_race_scan_finds_the_pattern():
    # the scan itself, on a listing with the pattern and on the same listing with the wait
    bad = """0000000000001000 <kern>:
	ds_read_b128 v[0:3], v4
	s_waitcnt vmcnt(14)
	s_barrier
	buffer_load_dwordx4 v5, s[8:11], 0 offen lds
"""
    good = bad.replace("\ts_barrier", "\ts_waitcnt lgkmcnt(0)\n\ts_barrier")
    assert lds_reads_pending_at_dma_barriers(bad) == {"kern": 1}
    assert lds_reads_pending_at_dma_barriers(good) == {}
