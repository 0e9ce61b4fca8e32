"""gfx950 disassembly of this repository's own HIP sources, for tests that
check properties of the generated code.  The built object in
runtimed_amd/_build is used when it is at least as new as its source and
the headers it may include (the build stamps objects with the time their
compile started); otherwise the source is compiled afresh (a few minutes
for the largest files)."""
import re
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "runtimed_amd" / "csrc"
BUILT = ROOT / "runtimed_amd" / "_build"
HIPCC = Path("/opt/rocm/bin/hipcc")
LLVM = Path("/opt/rocm/llvm/bin")
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"
HAVE_TOOLS = HIPCC.exists() and (LLVM / "llvm-objdump").exists() and (LLVM / "clang-offload-bundler").exists()


def _fresh(obj: Path, src: Path) -> bool:
    if not obj.exists():
        return False
    deps = [src, *CSRC.glob("*.h"), *(ROOT / "include").glob("*.h")]
    return all(d.stat().st_mtime <= obj.stat().st_mtime for d in deps)


def disassembly(src_name: str, tmp: Path) -> list:
    src = CSRC / src_name
    obj = BUILT / (src.stem + ".o")
    if not _fresh(obj, src):
        obj = tmp / (src.stem + ".o")
        subprocess.run([str(HIPCC), "-O3", "-std=c++17", "--offload-arch=gfx950", "-Xclang", "-target-feature",
                        "-Xclang", "-packed-fp32-ops", "-x", "hip", "-c", str(src), "-o", str(obj)],
                       check=True, capture_output=True)
    fatbin = tmp / (src.stem + ".fatbin")
    subprocess.run([str(LLVM / "llvm-objcopy"), f"--dump-section=.hip_fatbin={fatbin}", str(obj),
                    str(tmp / (src.stem + ".stripped.o"))], check=True, capture_output=True)
    hsaco = tmp / (src.stem + ".hsaco")
    subprocess.run([str(LLVM / "clang-offload-bundler"), "--type=o", f"--input={fatbin}", "--unbundle",
                    f"--targets={TARGET}", f"--output={hsaco}"], check=True, capture_output=True)
    return subprocess.run([str(LLVM / "llvm-objdump"), "-d", "--mcpu=gfx950", str(hsaco)], check=True,
                          capture_output=True, text=True).stdout.splitlines()


def kernels(lines: list, pattern: str) -> dict:
    """Mangled name -> its instruction lines (encodings and comments cut),
    for every function whose name matches `pattern`."""
    starts = [(i, m.group(1)) for i, l in enumerate(lines) if (m := re.match(r"^[0-9a-f]+ <(\S+)>:", l))]
    starts.append((len(lines), ""))
    out = {}
    for (a, name), (b, _) in zip(starts, starts[1:]):
        if re.search(pattern, name):
            body = []
            for l in lines[a + 1:b]:
                ins = l.split("//")[0].split(";")[0].strip()
                if ins and not ins.endswith(":"):
                    body.append(ins)
            out[name] = body
    return out
