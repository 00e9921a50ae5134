"""In-tree build of libgt_attn.so (hipcc, gfx950).

    python gguf_train_amd/_build.py            (a script: the package needs the library)

Objects go to gguf_train_amd/_build/ (ignored by git); the shared library is written next to
this file so that it travels with the source tree.  (The test-only CPU oracle has its own
build, oracle/build.py.)
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
OBJ_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "libgt_attn.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-fvisibility=hidden",
    "-Wall",
    "-Wno-unused-function",
    # packed fp32 VALU ops stay off: the compiler must not form v_pk_{add,mul,fma}_f32
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _sources() -> list[Path]:
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def _source_hash() -> str:
    # loaded by path: importing the package would load the library being built
    import importlib.util

    spec = importlib.util.spec_from_file_location("_gt_srchash", PKG_DIR / "_srchash.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.source_hash(PKG_DIR)


def _generate() -> None:
    """Generated sources (into the object directory, which the compiles search): the pipelined
    prefill kernel's assembly body."""
    gen = CSRC / "prefill_asm_gen.py"
    proc = subprocess.run([sys.executable, str(gen), str(OBJ_DIR / "prefill_asm_body.inc")], capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"{gen.name} failed:\n{proc.stdout}\n{proc.stderr}")


def _compile(src: Path, digest: str) -> Path:
    obj = OBJ_DIR / (src.name + ".o")
    cmd = [HIPCC, *HIP_FLAGS, f'-DGT_SOURCE_HASH="{digest}"', f"-I{OBJ_DIR}", "-x", "hip", "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    # the host pass does not know the gfx feature flag; everything else is worth showing
    noise = "is not a recognized feature for this target"
    msg = "\n".join(l for l in (proc.stderr or "").splitlines() if noise not in l).strip()
    if msg:
        print(f"[gt_attn build] {src.name}:\n{msg}", file=sys.stderr)
    return obj


def build_library(jobs: int | None = None) -> Path:
    OBJ_DIR.mkdir(exist_ok=True)
    _generate()
    srcs = _sources()
    jobs = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    digest = _source_hash()
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, digest), srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def main(argv: list[str]) -> int:
    print(f"[gt_attn build] {build_library()}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main(sys.argv[1:]))
