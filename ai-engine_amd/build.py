"""Build libpagedkv.so (HIP for gfx950) in-tree with hipcc.

Usage: python ai-engine_amd/build.py [-j N]

Every source in csrc/ is compiled to an object under _build/ and linked into
ai-engine_amd/libpagedkv.so.  Objects are rebuilt when the source or a
header is newer, but ``build(force=True)`` (what __graft_entry__.build()
calls) always recompiles everything.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libpagedkv.so")
ROOT = os.path.dirname(HERE)

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

SOURCES = [
    "pkv_capi.cpp",
    "block_table.cpp",
    "compact_plan.cpp",
    "pkv_sched.cpp",
    "pkv_kvcopy.hip",
    "pkv_decode.hip",
    "pkv_prefill.hip",
    "pkv_mixed.hip",
    "pkv_rope.hip",
    "pkv_sample.hip",
]

# Packed-FP32 instructions stay off (the compiler would otherwise form
# v_pk_fma_f32 and friends from ordinary float code).
COMMON = [
    "-O3", "-fPIC", "-std=c++17", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result",
    f"-I{os.path.join(ROOT, 'include')}",
]


# Per-source extras.  Prefill keeps its MFMA accumulators in ordinary VGPRs
# (no AGPR round trips for the softmax rescale; measured faster on gfx950);
# so does the mixed launch, which runs the same prefill body.
EXTRA = {
    "pkv_prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "pkv_mixed.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _headers() -> list[str]:
    hs = [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".h")]
    hs.append(os.path.join(ROOT, "include", "pagedkv.h"))
    return hs


def _obj(src: str) -> str:
    return os.path.join(BUILD, src + ".o")


def _stale(src: str, hdr_mtime: float) -> bool:
    o = _obj(src)
    if not os.path.exists(o):
        return True
    om = os.path.getmtime(o)
    return om < os.path.getmtime(os.path.join(CSRC, src)) or om < hdr_mtime


def _compile(src: str) -> tuple[str, int, str]:
    cmd = [HIPCC, *COMMON, *EXTRA.get(src, [])]
    if src.endswith(".hip"):
        cmd += ["-x", "hip"]
    cmd += ["-c", os.path.join(CSRC, src), "-o", _obj(src)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    return src, r.returncode, (r.stdout + r.stderr)


def build(force: bool = False, jobs: int = 8, verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    hdr_mtime = max(os.path.getmtime(h) for h in _headers())
    todo = [s for s in SOURCES if force or _stale(s, hdr_mtime)]
    if todo:
        with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
            for src, rc, out in ex.map(_compile, todo):
                # hipcc's host pass does not know the packed-fp32 feature
                # name and warns about it; that warning is expected.
                lines = [l for l in out.splitlines() if "packed-fp32-ops" not in l]
                if rc != 0:
                    sys.stderr.write("\n".join(lines) + "\n")
                    raise RuntimeError(f"hipcc failed on {src}")
                if verbose and lines:
                    sys.stderr.write("\n".join(lines) + "\n")
    if todo or not os.path.exists(LIB):
        tmp = LIB + ".tmp"
        cmd = [HIPCC, "-shared", f"--offload-arch={ARCH}", "-o", tmp,
               *[_obj(s) for s in SOURCES]]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            sys.stderr.write(r.stdout + r.stderr)
            raise RuntimeError("link of libpagedkv.so failed")
        os.replace(tmp, LIB)
    return LIB


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=8)
    ap.add_argument("--force", action="store_true")
    ap.add_argument("-v", action="store_true")
    a = ap.parse_args()
    print(build(force=a.force, jobs=a.j, verbose=a.v))


if __name__ == "__main__":
    main()
