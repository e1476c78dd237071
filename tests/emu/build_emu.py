"""Builds the CPU emulation library of the product's kernels (TEST INFRASTRUCTURE ONLY).

The product's tinyserve_amd/csrc/*.hip sources are compiled as host C++ against the stand-in HIP
environment of tests/emu/emu_hip.h (fiber-per-thread execution, cross-lane operations and the
matrix-core instruction evaluated on the CPU). Textual adaptations are made on copies of the
sources, never on the sources themselves: the dynamic LDS declaration becomes a pointer to the
emulated LDS; each static __shared__ declaration becomes a reference into the emulated
workgroup's LDS arena (which, like the dynamic LDS, starts every workgroup as garbage); and the
inline-assembly idioms the tile kernel uses (a register copy that places a wait, an LDS-wait +
workgroup barrier, which does not wait for global->LDS loads, and an empty statement that hides
a value from the optimiser) become their host equivalents. Any other inline assembly or __shared__ form stops the build.

The result, tests/emu/_build/libtsm_emu[_asan|_tsan].so, exports the same C ABI as
libtinyserve_moe.so and is loaded only by tests. With sanitizer="asan" every memory access of the
kernels is checked by AddressSanitizer (the CPU counterpart of a GPU memory fault); with
sanitizer="tsan" the kernels run under ThreadSanitizer with the GPU's happens-before edges only
(data races between wavefronts and workgroups).
"""
import hashlib
import os
import re
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
CSRC = os.path.join(ROOT, "tinyserve_amd", "csrc")
OUT = os.path.join(HERE, "_build")

ASM_REWRITES = [
    (re.compile(r'asm volatile\("v_mov_b32 %0, %1" : "=v"\((\w+)\) : "v"\((\w+)\)\);'),
     r"\1 = \2;"),
    (re.compile(r'asm volatile\("s_waitcnt lgkmcnt\(0\)\\n\\ts_barrier" ::: "memory"\);'),
     "::emu::s_barrier();"),
    # an empty asm that only hides a value from the optimiser: nothing to do on the host
    (re.compile(r'asm volatile\(""\s*:\s*"\+[sv]"\((\w+)\)\);'), r"(void)\1;"),
]
FLAGS = ["-std=c++17", "-O2", "-g", "-fPIC", "-fno-omit-frame-pointer", "-w", "-mavx2", "-mfma"]
LDS_DECL = re.compile(r"extern __shared__[^;]*\bchar (\w+)\[\];")


def _clang():
    for c in ("/opt/rocm/llvm/bin/clang++", shutil.which("clang++") or ""):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("clang++ not found")


STATIC_LDS = re.compile(
    r"__shared__\s+((?:__attribute__\(\([^;]*?\)\)\s+)*)([A-Za-z_][\w:]*)\s+([^;]+);")
DECLARATOR = re.compile(r"(\w+)\s*((?:\[[^\]]*\])*)$")


def _static_lds(m: re.Match, keys: list) -> str:
    """`__shared__ T a[n][m], b;` -> references into the emulated workgroup's LDS arena, which
    starts every workgroup as garbage (on the GPU LDS is not initialised, and a workgroup does not
    see the previous one's)."""
    attrs, ty, decls = m.group(1), m.group(2), m.group(3)
    al = re.search(r"aligned\((\d+)\)", attrs)
    align = f"alignof({ty})" if not al else f"({al.group(1)} > alignof({ty}) ? {al.group(1)} : alignof({ty}))"
    out = []
    for d in decls.split(","):
        dm = DECLARATOR.match(d.strip())
        if not dm:
            raise RuntimeError(f"unrecognised __shared__ declarator {d!r}")
        name, dims = dm.group(1), dm.group(2)
        keys.append(name)
        key = len(keys)
        if dims:
            out.append(f"{ty} (&{name}){dims} = *reinterpret_cast<{ty}(*){dims}>("
                       f"::emu::static_lds({key}, sizeof({ty}{dims}), {align}));")
        else:
            out.append(f"{ty}& {name} = *reinterpret_cast<{ty}*>("
                       f"::emu::static_lds({key}, sizeof({ty}), {align}));")
    return " ".join(out)


def adapt(text: str, name: str, keys: list) -> str:
    text = LDS_DECL.sub(r"char* const \1 = ::emu::dynamic_lds();", text)
    text = STATIC_LDS.sub(lambda m: _static_lds(m, keys), text)
    if "__shared__" in text:
        raise RuntimeError(f"{name}: a __shared__ declaration the emulator does not know")
    for pat, rep in ASM_REWRITES:
        text = pat.sub(rep, text)
    if re.search(r"\b(asm|__asm__)\s*(volatile\s*)?\(", text):
        raise RuntimeError(f"{name}: inline assembly the emulator does not know")
    return text


def sources():
    return sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))


SANITIZERS = (None, "asan", "tsan")


def build(sanitizer: str = None, jobs: int = 8) -> str:
    if sanitizer not in SANITIZERS:
        raise ValueError(f"sanitizer must be one of {SANITIZERS}")
    tag = f"_{sanitizer}" if sanitizer else ""
    lib = os.path.join(OUT, f"libtsm_emu{tag}.so")
    h = hashlib.sha256()
    inputs = [os.path.join(CSRC, f) for f in sources()] + [
        os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".h")] + [
        os.path.join(HERE, "emu_hip.h"), os.path.join(HERE, "emu_runtime.cpp"),
        os.path.join(ROOT, "include", "tinyserve_moe.h"), os.path.abspath(__file__)]
    for p in sorted(inputs):
        h.update(open(p, "rb").read())
    h.update((" ".join(FLAGS) + tag).encode())
    stamp = lib + ".sha256"
    if os.path.exists(lib) and os.path.exists(stamp) and open(stamp).read() == h.hexdigest():
        return lib
    src_dir = os.path.join(OUT, "src")
    obj_dir = os.path.join(OUT, f"obj{tag}")
    os.makedirs(src_dir, exist_ok=True)
    os.makedirs(obj_dir, exist_ok=True)
    flags = FLAGS + [f"-I{os.path.join(HERE, 'include')}", f"-I{os.path.join(ROOT, 'include')}",
                     f"-I{CSRC}", "-include", os.path.join(HERE, "emu_hip.h")]
    runtime_flags = list(flags)
    if sanitizer:
        # -O1: the sanitizer instrumentation at -O2 takes tens of minutes on the router unit
        flags = [f for f in flags if f != "-O2"] + ["-O1"]
        runtime_flags = list(flags)
    if sanitizer == "asan":
        flags += ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined"]
        runtime_flags = list(flags)
    elif sanitizer == "tsan":
        # the kernels are instrumented; the runtime is not (its scheduler state is shared by
        # every fiber by design) and reports its own accesses on the kernels' behalf
        flags += ["-fsanitize=thread"]
        runtime_flags += ["-DEMU_TSAN"]
    units = []
    keys = []
    for f in sources():
        dst = os.path.join(src_dir, f[:-4] + ".cpp")
        text = adapt(open(os.path.join(CSRC, f)).read(), f, keys)
        if not os.path.exists(dst) or open(dst).read() != text:
            open(dst, "w").write(text)
        units.append(dst)
    units.append(os.path.join(HERE, "emu_runtime.cpp"))
    cxx = _clang()

    runtime = units[-1]

    def compile_one(src):
        obj = os.path.join(obj_dir, os.path.basename(src) + ".o")
        fl = runtime_flags if src == runtime else flags
        r = subprocess.run([cxx, *fl, "-c", src, "-o", obj], capture_output=True, text=True)
        if r.returncode:
            raise RuntimeError(f"emulation build of {src} failed:\n{r.stderr[-4000:]}")
        return obj

    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, units))
    link = [cxx, "-shared", "-o", lib + ".tmp", *objs]
    if sanitizer == "asan":
        link.insert(1, "-fsanitize=address,undefined")
    elif sanitizer == "tsan":
        link.insert(1, "-fsanitize=thread")
    r = subprocess.run(link, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"emulation link failed:\n{r.stderr[-4000:]}")
    os.replace(lib + ".tmp", lib)
    open(stamp, "w").write(h.hexdigest())
    return lib


if __name__ == "__main__":
    san = next((a[2:] for a in sys.argv[1:] if a in ("--asan", "--tsan")), None)
    print(build(san))
