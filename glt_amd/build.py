"""Build libglt.so (gfx950) in-tree from glt_amd/csrc/*.hip.

Usage: python -m glt_amd.build   (or glt_amd.build.build())
Every HIP source is compiled for gfx950 only, then linked into
glt_amd/libglt.so next to this file.
"""
import concurrent.futures
import os
import re
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libglt.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    "-std=c++17", "-O3", "-fPIC", f"--offload-arch={ARCH}",
    # packed-f32 VALU forms are kept out of the generated code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
    # per-kernel register / scratch report, checked below
    "-Rpass-analysis=kernel-resource-usage",
]
_RE_NAME = re.compile(r"remark: Function Name: (\S+)")
_RE_SCRATCH = re.compile(r"remark:\s+ScratchSize \[bytes/lane\]: (\d+)")


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


_RE_VREG = re.compile(r"v\[(\d+):(\d+)\]|v(\d+)$")
_RE_STORE = re.compile(r"(buffer_store_dwordx[34]|global_store_dwordx[34])\s+(\S+?),\s*(\S+?),")


def _vregs(spec):
    m = _RE_VREG.match(spec)
    if not m:
        return set()
    if m.group(3) is not None:
        return {int(m.group(3))}
    return set(range(int(m.group(1)), int(m.group(2)) + 1))


def store_data_hazards(asm_text):
    """Places in gfx950 assembly where a vector-memory store of more than 8
    bytes is followed, within two wait states, by a VALU write of one of its
    data registers. The hardware needs two wait states there (without them
    the store sends the new value); the compiler omits them for buffer
    stores with a register scalar offset. Returns (line, store, writer)."""
    lines = asm_text.splitlines()
    out = []
    for i, line in enumerate(lines):
        st = line.split(";")[0].strip()
        m = _RE_STORE.match(st)
        if not m:
            continue
        data = _vregs(m.group(2) if m.group(1).startswith("buffer") else m.group(3))
        ws, j = 0, i + 1
        while j < len(lines) and ws < 2:
            t = lines[j].split(";")[0].strip()
            j += 1
            if not t or t.startswith(".") or t.endswith(":"):
                continue
            n = re.match(r"s_nop\s+(\d+)", t)
            if n:
                ws += int(n.group(1)) + 1
                continue
            w = re.match(r"(v_\S+)\s+(v\[\d+:\d+\]|v\d+)", t)
            if w and not w.group(1).startswith(("v_cmp", "v_readfirstlane", "v_readlane")) and _vregs(w.group(2)) & data:
                out.append((i + 1, st, t))
                break
            ws += 1
    return out


def _check_assembly(src):
    """Compiles src's device code to assembly and rejects store-data hazards."""
    asm = os.path.join(BUILD, os.path.basename(src) + ".s")
    cmd = [HIPCC, *[f for f in FLAGS if f not in ("-fPIC", "-Rpass-analysis=kernel-resource-usage")],
           "--cuda-device-only", "-S", src, "-o", asm]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc -S failed for {src}:\n{r.stdout}\n{r.stderr}")
    bad = store_data_hazards(open(asm).read())
    if bad:
        raise RuntimeError(f"{os.path.basename(src)}: {len(bad)} store-data hazard(s), first at line {bad[0][0]} "
                           f"of {asm}: {bad[0][1]} / {bad[0][2]}")


def _compile(src):
    _check_assembly(src)
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [HIPCC, *FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    # No kernel may use scratch: in these kernels it only ever appears as a
    # register spill or a copied argument block, both silent slowdowns.
    name = None
    for line in r.stderr.splitlines():
        m = _RE_NAME.search(line)
        if m:
            name = m.group(1)
            continue
        m = _RE_SCRATCH.search(line)
        if m and int(m.group(1)) > 0:
            raise RuntimeError(f"{os.path.basename(src)}: kernel {name} uses {m.group(1)} bytes/lane of scratch")
    return obj


def build(verbose=False):
    if shutil.which(HIPCC) is None and not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    r = subprocess.run([HIPCC, "-shared", f"--offload-arch={ARCH}", "-o", tmp, *objs],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
