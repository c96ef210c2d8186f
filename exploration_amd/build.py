"""Build ``libst_attn.so`` (HIP kernels for gfx950 + the C ABI) in-tree.

``python -m exploration_amd.build`` compiles every ``csrc/*.hip`` with hipcc
in parallel and links them into ``exploration_amd/libst_attn.so``. Always
rebuilds (object files are cached by content hash under ``_build/``).
"""
import concurrent.futures
import hashlib
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
OUT = os.path.join(HERE, "libst_attn.so")
BUILD = os.path.join(HERE, "_build")

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-fPIC",
    # no packed fp32 instructions anywhere in the device code, and no
    # mixed-precision VOP3P forms either (v_fma_mix*/v_mad_mix*: fp32 FMAs
    # with fp16 operands or half-register fp16 results, which hipcc otherwise
    # folds the fp16 conversions into). Both belong to the packed-math
    # datapath whose results have not been reliable on this platform: dQ
    # fragments assembled from v_fma_mix{lo,hi}_f16 writes came out wrong at
    # fp16, head_dim 64, block 8, while the same kernel with separate FMA and
    # conversion instructions is exact. bf16 code never uses them.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Xclang", "-target-feature", "-Xclang", "-fma-mix-insts",
    # no NaN inputs are meaningful here: without IEEE mode, v_max/v_min need
    # no canonicalising copy of each operand (one VALU op per max saved)
    "-fno-honor-nans", "-mno-amdgpu-ieee",
    "-Wno-pass-failed",
]


# Per-source extra flags. The pipelined dense kernels keep their score tiles
# in VGPRs (MFMA results feed the softmax directly, no AGPR round trip; for
# the dQ kernel this also removes its scratch spills).
EXTRA_FLAGS = {
    "dense_fwd_fast.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "dense_bwd_fast.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _sources():
    return sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))


def _digest(src):
    h = hashlib.sha256()
    h.update(" ".join([HIPCC] + FLAGS + EXTRA_FLAGS.get(src, [])).encode())
    for name in sorted(os.listdir(CSRC)):
        if name.endswith(".h") or name == src:
            with open(os.path.join(CSRC, name), "rb") as f:
                h.update(name.encode() + f.read())
    with open(os.path.join(INCLUDE, "st_attn.h"), "rb") as f:
        h.update(f.read())
    h.update(src.encode())
    return h.hexdigest()[:16]


def _compile(src):
    obj = os.path.join(BUILD, f"{src[:-4]}-{_digest(src)}.o")
    if os.path.exists(obj):
        return obj
    tmp = obj + ".tmp"
    cmd = [HIPCC] + FLAGS + EXTRA_FLAGS.get(src, []) + ["-c", os.path.join(CSRC, src), "-o", tmp]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{proc.stderr}")
    os.replace(tmp, obj)
    return obj


def build(verbose=True):
    """Compile and link the library; returns its path."""
    if not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    os.makedirs(BUILD, exist_ok=True)
    sources = _sources()
    workers = min(len(sources), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)), 8)
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = OUT + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, OUT)
    keep = {os.path.basename(o) for o in objs}
    for name in os.listdir(BUILD):
        if name.endswith(".o") and name not in keep:
            os.remove(os.path.join(BUILD, name))
    if verbose:
        print(f"built {OUT}", flush=True)
    return OUT


def clean():
    shutil.rmtree(BUILD, ignore_errors=True)
    if os.path.exists(OUT):
        os.remove(OUT)


if __name__ == "__main__":
    if "--clean" in sys.argv:
        clean()
    build()
