"""Build libhos_hip.so (gfx950) in-tree with hipcc.

Every .hip under hos_amd/csrc is compiled for gfx950 only and linked into
hos_amd/libhos_hip.so, the C-ABI library declared by include/hos_hip.h.
"""
import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libhos_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function",
    # packed-fp32 VALU forms are disabled on this pool (silent wrong results seen on some forms)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# Files whose f32 arithmetic must round once per operation (byte-exact GGUF codec): no fusion of a·b + c
# anywhere, including inside inlined header intrinsics.
NO_CONTRACT = {"quant.hip"}
# Files whose MFMA accumulators are read by VALU work every iteration (the attention softmax): keep them in
# VGPRs (the default AGPR form costs a read and a write per accumulator register around that work).
MFMA_VGPR = {"attention.hip"}


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


# Host-side AddressSanitizer + UndefinedBehaviorSanitizer build (CPU tests of the file parsers only; device code
# is compiled as usual, GPU sanitizers are not used): `python -m hos_amd.build --sanitize`.
SAN_FLAGS = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined", "-Xarch_host",
             "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer", "-g"]
SAN_BUILD = os.path.join(BUILD, "san")
SAN_LIB = os.path.join(SAN_BUILD, "libhos_hip.so")


def _compile(src, san=False):
    obj = os.path.join(SAN_BUILD if san else BUILD, os.path.basename(src) + ".o")
    extra = ["-ffp-contract=off"] if os.path.basename(src) in NO_CONTRACT else []
    if os.path.basename(src) in MFMA_VGPR:
        extra += ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]
    cmd = [HIPCC] + FLAGS + extra + (SAN_FLAGS if san else []) + ["-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


def build_sanitized(verbose=False):
    """libhos_hip.so with host code under ASan + UBSan, in _build/san/ (load it with HOS_HIP_LIB and
    LD_PRELOAD=asan_runtime())."""
    os.makedirs(SAN_BUILD, exist_ok=True)
    srcs = sources()
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, san=True), srcs))
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-fsanitize=address,undefined", "-o", SAN_LIB] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"sanitized link failed:\n{r.stderr}")
    if verbose:
        print(f"built {SAN_LIB}")
    return SAN_LIB


def asan_runtime():
    """The clang ASan runtime the sanitized library needs preloaded into an uninstrumented python."""
    r = subprocess.run([HIPCC.replace("hipcc", "amdclang++") if "hipcc" in HIPCC else "amdclang++",
                        "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
    path = r.stdout.strip()
    if not os.path.isabs(path):
        import glob
        found = glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so")
        path = found[0] if found else path
    return path


if __name__ == "__main__":
    if "--sanitize" in sys.argv:
        build_sanitized(verbose=True)
        print(asan_runtime())
    else:
        build(verbose=True)
    sys.exit(0)
