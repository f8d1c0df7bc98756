"""Builds the CPU-emulated C ABI (tests/emu/_build/libnc_emu.so) from the same kernel
sources as the gfx950 library, with g++ and the emulation shim in tests/emu/hip/.

With NC_EMU_SANITIZE=1 it builds libnc_emu_asan.so instead, under AddressSanitizer and
UndefinedBehaviorSanitizer (host code only: the emulator runs the kernels on the CPU), so an
out-of-bounds global access in a kernel source fails the emulated launch.  The Python
process must load the sanitizer runtime first:

    NC_EMU_SANITIZE=1 LD_PRELOAD=$(g++ -print-file-name=libasan.so) \
        ASAN_OPTIONS=detect_leaks=0 python -m pytest tests/test_emu_kernels.py
"""
import concurrent.futures as cf
import fcntl
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
CSRC = os.path.join(ROOT, "neurocell-v2_amd", "csrc")
SANITIZE = os.environ.get("NC_EMU_SANITIZE") == "1"
OUT_DIR = os.path.join(HERE, "_build_asan" if SANITIZE else "_build")
LIB = os.path.join(OUT_DIR, "libnc_emu_asan.so" if SANITIZE else "libnc_emu.so")
SOURCES = [os.path.join(CSRC, f) for f in ("nc_codd.hip", "nc_epilogue.hip", "nc_spectral.hip",
                                                   "nc_spectral_large.hip", "nc_direct.hip")]
FLAGS = ["g++", "-std=c++20", "-O1", "-fPIC", "-pthread", "-I", HERE]
# every report aborts the emulated launch (undefined behaviour included), so a test cannot pass
# over one
SAN = (["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer"]
       if SANITIZE else [])


def _stale() -> bool:
    if not os.path.exists(LIB):
        return True
    deps = SOURCES + [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".h")]
    deps += [os.path.join(HERE, "hip", "hip_runtime.h"), os.path.join(HERE, "emu_main.cpp"),
             os.path.join(ROOT, "include", "neurocell_hip.h")]
    t = os.path.getmtime(LIB)
    return any(os.path.getmtime(d) > t for d in deps)


def _obj(src):
    obj = os.path.join(OUT_DIR, os.path.basename(src) + ".o")
    lang = ["-x", "c++"] if src.endswith(".hip") else []
    subprocess.run(FLAGS + SAN + lang + ["-c", src, "-o", obj], check=True,
                   capture_output=True)
    return obj


def build() -> str:
    if not _stale():
        return LIB
    os.makedirs(OUT_DIR, exist_ok=True)
    # one builder at a time (parallel test workers share the build folder)
    with open(os.path.join(OUT_DIR, ".lock"), "w") as lock:
        fcntl.flock(lock, fcntl.LOCK_EX)
        if _stale():
            with cf.ThreadPoolExecutor(4) as ex:
                objs = list(ex.map(_obj, SOURCES + [os.path.join(HERE, "emu_main.cpp")]))
            subprocess.run(["g++", "-shared", "-pthread", *SAN, "-o", LIB + ".tmp", *objs],
                           check=True)
            os.replace(LIB + ".tmp", LIB)
    return LIB


if __name__ == "__main__":
    print(build())
