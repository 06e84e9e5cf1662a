"""The direct-to-LDS loads in gemm.hip, attention.hip and attention_bwd.hip
set M0 inside their inline asm without declaring it (the register is
reserved, so clang will not take it as a clobber).  That is safe only while
the compiler itself keeps nothing in M0 in those code objects.  This test
reads the AMD assembly of the code objects built here and checks exactly
that: every instruction naming M0 is one of the asm statements' own
`s_mov_b32 m0, sN`, each directly followed by its `global_load_lds_dwordx4`,
and no instruction that reads M0 implicitly (messages, GDS/GWS, relative
moves, interpolation, LDS-direct, buffer loads to LDS) appears anywhere.  A
toolchain that starts using M0 in these kernels fails here instead of
corrupting LDS at run time."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "bluewolf-plus-plus_amd", "lib")
LLVM = "/opt/rocm/llvm/bin"
KERNELS = ["gemm", "attention", "attention_bwd", "attention_f32", "grad", "rowops"]
# instructions that read M0 without naming it
IMPLICIT = re.compile(r"\b(s_sendmsg\w*|s_movrel\w*|v_movrel\w*|ds_gws\w*|ds_ordered\w*|ds_append|ds_consume|"
                      r"v_interp\w*|ds_param\w*|ds_direct\w*|s_set_gpr_idx\w*|buffer_load\w*\s.*\blds\b|"
                      r"buffer_store_lds\w*|global_load_lds_(?!dwordx4)\w*)")


def _asm(kernel, tmp_path):
    bundle = os.path.join(LIB, f"bwpp_{kernel}.hsaco")
    bundler, objdump = os.path.join(LLVM, "clang-offload-bundler"), os.path.join(LLVM, "llvm-objdump")
    if not (os.path.exists(bundle) and shutil.which(bundler) and shutil.which(objdump)):
        pytest.skip("code object or ROCm LLVM tools not present")
    obj = tmp_path / f"{kernel}.o"
    subprocess.run([bundler, "--unbundle", "--type=o", f"--input={bundle}",
                    "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--output={obj}"], check=True)
    out = subprocess.run([objdump, "-d", "--mcpu=gfx950", str(obj)], check=True, capture_output=True, text=True)
    lines = []
    for ln in out.stdout.splitlines():
        ins = ln.split("//", 1)[0].strip()
        if ins and not ins.endswith(":") and not ins.startswith("Disassembly") and "file format" not in ins:
            lines.append(ins)
    return lines


@pytest.mark.parametrize("kernel", KERNELS)
def test_m0_written_only_by_lds_dma_asm(kernel, tmp_path):
    lines = _asm(kernel, tmp_path)
    assert len(lines) > 100, "disassembly looks empty"
    moves = dmas = 0
    for i, ins in enumerate(lines):
        assert not IMPLICIT.search(ins), f"{kernel}: instruction reads M0 implicitly: {ins}"
        if re.search(r"\bm0\b", ins):
            assert re.match(r"s_mov_b32 m0, s\d+$", ins), f"{kernel}: M0 used outside the LDS-DMA asm: {ins}"
            assert i + 1 < len(lines) and lines[i + 1].startswith("global_load_lds_dwordx4"), \
                f"{kernel}: M0 write not followed by its LDS DMA: {ins} / {lines[i + 1] if i + 1 < len(lines) else ''}"
            moves += 1
        if ins.startswith("global_load_lds_dwordx4"):
            assert i > 0 and lines[i - 1].startswith("s_mov_b32 m0,"), f"{kernel}: LDS DMA without its M0 write"
            dmas += 1
    assert moves == dmas
    if kernel in ("gemm", "attention", "attention_bwd"):
        assert dmas > 0, f"{kernel}: expected the LDS-DMA asm in this code object"
