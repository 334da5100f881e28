"""Every kernel of the built library runs without scratch memory: no private
segment, no VGPR or SGPR spills. A kernel that indexes a by-value argument
struct at run time after writing to it gets a scratch copy of the struct (the
board-layout GEMVs once did, and the gemv2 LM head took 60 us instead of 35);
spills would show up the same way. Reads the code-object metadata of this
repository's own build (CPU only)."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "llm-kv260_amd", "libkv260gemv.so")
PLAN_CO = os.path.join(ROOT, "llm-kv260_amd", "_build", "chain_plan.co")
LLVM = "/opt/rocm/llvm/bin"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"


def _tool(name):
    path = os.path.join(LLVM, name)
    return path if os.path.exists(path) else shutil.which(name)


def _kernels(code_object):
    """(name, private segment bytes, VGPR spills, SGPR spills) per kernel."""
    notes = subprocess.run([_tool("llvm-readelf"), "--notes", code_object], capture_output=True, text=True,
                           check=True).stdout
    out = []
    for block in notes.split("  - .")[1:]:
        name = re.search(r"\.name:\s+(\S+)", block)
        priv = re.search(r"\.private_segment_fixed_size:\s+(\d+)", block)
        if not (name and priv):
            continue
        vsp = re.search(r"\.vgpr_spill_count:\s+(\d+)", block)
        ssp = re.search(r"\.sgpr_spill_count:\s+(\d+)", block)
        out.append((name.group(1), int(priv.group(1)), int(vsp.group(1)) if vsp else 0,
                    int(ssp.group(1)) if ssp else 0))
    return out


def _library_code_objects(tmp_path):
    """The gfx950 code objects of the library's offload bundles (one per translation unit)."""
    fatbin = tmp_path / "fatbin.bin"
    subprocess.run(["objcopy", f"--dump-section=.hip_fatbin={fatbin}", LIB, str(tmp_path / "lib.so")], check=True,
                   capture_output=True)
    data = fatbin.read_bytes()
    starts = [m.start() for m in re.finditer(re.escape(MAGIC), data)]
    cos = []
    for i, s in enumerate(starts):
        end = starts[i + 1] if i + 1 < len(starts) else len(data)
        part = tmp_path / f"b{i}.bin"
        part.write_bytes(data[s:end])
        co = tmp_path / f"c{i}.co"
        r = subprocess.run([_tool("clang-offload-bundler"), "--unbundle", "--type=o", f"--input={part}",
                            f"--targets={TARGET}", f"--output={co}"], capture_output=True, text=True)
        if r.returncode == 0 and co.stat().st_size > 0:
            cos.append(str(co))
    return cos


@pytest.mark.skipif(not os.path.exists(LIB), reason="library not built")
def test_no_kernel_uses_scratch(tmp_path):
    if not (shutil.which("objcopy") and _tool("clang-offload-bundler") and _tool("llvm-readelf")):
        pytest.skip("objcopy / clang-offload-bundler / llvm-readelf not available")
    cos = _library_code_objects(tmp_path)
    if os.path.exists(PLAN_CO):
        cos.append(PLAN_CO)
    kernels = [k for co in cos for k in _kernels(co)]
    assert len(kernels) > 50, f"only {len(kernels)} kernels found"
    assert any("gemv_m1_kernel" in k[0] for k in kernels)
    bad = [k for k in kernels if k[1] or k[2] or k[3]]
    assert not bad, "kernels with scratch (name, private bytes, VGPR spills, SGPR spills): " + repr(bad)
