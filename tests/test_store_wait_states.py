"""Buffer stores of more than 8 bytes never carry a register scalar offset
(no GPU needed: the check reads the gfx950 code object inside the built
library).

A MUBUF store with more than 8 bytes of data needs one wait state before an
instruction overwrites its data VGPRs. The GCN rule the compiler applies
exempts stores whose scalar offset is an SGPR, so it emits none for them
(`buffer_store_dwordx4 v[4:7], v30, s[0:3], s8 offen` followed directly by
`v_mul_f32 v7, ...`), and on gfx950 such a store wrote the overwritten
values: wrong results, no fault. The library's 16-byte store helper
therefore folds the scalar part into the lane offset; this test disassembles
every kernel of libcubutterfly.so and fails on any 12- or 16-byte buffer
store whose scalar-offset operand is an SGPR. A planted store of that form,
compiled here, shows that the scan finds one."""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROCM_LLVM = Path("/opt/rocm/llvm/bin")
LIB = Path(__file__).resolve().parents[1] / "cubutterfly_amd" / "libcubutterfly.so"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"
WIDE_STORE = re.compile(r"\b(buffer_store_dwordx[34]|buffer_store_b(?:96|128))\s+v\[\d+:\d+\],\s*\S+,\s*s\[\d+:\d+\],"
                        r"\s*(\S+)")

pytestmark = pytest.mark.skipif(not (ROCM_LLVM / "llvm-objdump").exists() or shutil.which("objcopy") is None,
                                reason="needs ROCm's llvm-objdump and binutils' objcopy")


def code_objects(binary, tmp_path):
    """gfx950 code objects of every offload bundle in a host binary's .hip_fatbin."""
    fatbin = tmp_path / "fatbin.bin"
    subprocess.run(["objcopy", "--dump-section", f".hip_fatbin={fatbin}", str(binary)], check=True,
                   capture_output=True)
    data = fatbin.read_bytes()
    magic = b"__CLANG_OFFLOAD_BUNDLE__"
    starts = [m.start() for m in re.finditer(re.escape(magic), data)] + [len(data)]
    objects = []
    for k in range(len(starts) - 1):
        bundle, obj = tmp_path / f"b{k}.bin", tmp_path / f"c{k}.o"
        bundle.write_bytes(data[starts[k]:starts[k + 1]])
        subprocess.run([str(ROCM_LLVM / "clang-offload-bundler"), "--unbundle", "--type=o", f"--targets={TARGET}",
                        f"--input={bundle}", f"--output={obj}"], check=True, capture_output=True)
        objects.append(obj)
    return objects


def wide_stores_with_sgpr_offset(obj):
    text = subprocess.run([str(ROCM_LLVM / "llvm-objdump"), "-d", "--mcpu=gfx950", str(obj)], check=True,
                          capture_output=True, text=True).stdout
    stores = [m for m in WIDE_STORE.finditer(text)]
    return len(stores), [m.group(0) for m in stores if re.fullmatch(r"s\d+", m.group(2))]


def test_library_has_no_wide_store_with_register_scalar_offset(tmp_path):
    assert LIB.exists(), "build the library first (python -m cubutterfly_amd.build)"
    total, bad = 0, []
    for obj in code_objects(LIB, tmp_path):
        n, found = wide_stores_with_sgpr_offset(obj)
        total += n
        bad += found
    assert total > 0, "no 16-byte buffer stores found: the scan no longer matches the disassembly"
    assert not bad, f"{len(bad)} wide stores with an SGPR scalar offset, e.g. {bad[:3]}"


def test_scan_finds_a_planted_register_scalar_offset(tmp_path):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    src = tmp_path / "planted.hip"
    src.write_text(
        "#include <hip/hip_runtime.h>\n"
        "__global__ void planted(float* out, unsigned n, unsigned off) {\n"
        "    __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(out, 0, int(n * 4), 0x00020000);\n"
        "    using V4 = __attribute__((ext_vector_type(4))) unsigned;\n"
        "    __builtin_amdgcn_raw_buffer_store_b128(V4{1u, 2u, 3u, threadIdx.x}, r, int(threadIdx.x * 16u),\n"
        "                                           int(off), 0);\n"
        "}\n")
    so = tmp_path / "planted.so"
    subprocess.run([hipcc, "--offload-arch=gfx950", "-O3", "-fPIC", "-shared", str(src), "-o", str(so)], check=True,
                   capture_output=True)
    found = [s for obj in code_objects(so, tmp_path) for s in wide_stores_with_sgpr_offset(obj)[1]]
    assert found, "the scan missed a 16-byte store with an SGPR scalar offset"
