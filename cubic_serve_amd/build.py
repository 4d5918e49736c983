"""Build the gfx950 HIP library in-tree: cubic_serve_amd/_lib/libcubic_mi355x.so.

hipcc cross-compiles on a machine without a GPU.  Flags:
  -ffp-contract=off   the Cubic decoder and acceptance transform are unfused IEEE
  -Xclang -target-feature -Xclang -packed-fp32-ops   no packed FP32 instructions
  -mllvm -amdgpu-mfma-vgpr-form   MFMA accumulators in VGPRs (no AGPR copies)
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
CSRC = PACKAGE / "csrc"
LIB_DIR = PACKAGE / "_lib"
LIB = LIB_DIR / "libcubic_mi355x.so"
SOURCES = ("cubic_capi.hip", "cubic_gemm.hip", "cubic_panel.hip", "cubic_accept.hip", "cubic_embed.hip", "cubic_moe.hip",
           "cubic_greedy.hip")
ARCH = "gfx950"
# Per-source flags.  The acceptance kernel sizes its LDS for three workgroups
# per CU (three waves per SIMD at its register count); LLVM's promotion of
# small private arrays to LDS would add 3 KB per workgroup and leave room for
# two, so that promotion is off for this file (the arrays stay in registers).
FILE_FLAGS = {"cubic_accept.hip": ("-mllvm", "-disable-promote-alloca-to-lds")}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the Cubic MI355X library needs ROCm's hipcc")


def flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-mllvm", "-amdgpu-mfma-vgpr-form",
        "-fvisibility=hidden", "-Wall", "-Wno-unused-function",
        f"-I{ROOT / 'include'}", f"-I{CSRC}",
    ]


def resource_usage(remarks: str) -> dict[str, dict[str, int]]:
    """Per-kernel counters from clang's kernel-resource-usage remarks."""
    usage: dict[str, dict[str, int]] = {}
    name = None
    for line in remarks.splitlines():
        if "remark:" not in line:
            continue
        text = line.split("remark:", 1)[1].split("[-Rpass", 1)[0].strip()
        if text.startswith("Function Name:"):
            name = text.split(":", 1)[1].strip()
            usage[name] = {}
        elif name and ":" in text:
            key, val = (t.strip() for t in text.rsplit(":", 1))
            if val.lstrip("-").isdigit():
                usage[name][key] = int(val)
    return usage


def build(verbose: bool = False, jobs: int = 3) -> Path:
    """Compile every HIP source (in parallel) and link the shared library."""
    LIB_DIR.mkdir(exist_ok=True)
    obj_dir = LIB_DIR / "obj"
    obj_dir.mkdir(exist_ok=True)
    cc = hipcc()
    procs = []
    objects = []
    for src in SOURCES:
        obj = obj_dir / (Path(src).stem + ".o")
        objects.append(obj)
        cmd = [cc, *flags(), *FILE_FLAGS.get(src, ()), "-Rpass-analysis=kernel-resource-usage",
               "-c", str(CSRC / src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        # output to a file, not a pipe: the resource remarks run to megabytes,
        # and a child blocked on a full pipe never exits
        log = tempfile.TemporaryFile()
        procs.append((src, subprocess.Popen(cmd, stdout=log, stderr=subprocess.STDOUT), log))
        while sum(p.poll() is None for _, p, _ in procs) >= jobs:
            procs[[p.poll() is None for _, p, _ in procs].index(True)][1].wait()
    failed = []
    usage: dict[str, dict[str, int]] = {}
    for src, p, log in procs:
        p.wait()
        log.seek(0)
        out = log.read().decode(errors="replace")
        log.close()
        usage.update(resource_usage(out))
        lines = [l for l in out.splitlines()
                 if "packed-fp32-ops" not in l and "kernel-resource-usage" not in l and "remark" not in l]
        if p.returncode != 0:
            failed.append((src, "\n".join(lines)))
        elif verbose and any(l.strip() for l in lines):
            print("\n".join(lines))
    if failed:
        raise RuntimeError("HIP build failed:\n" + "\n\n".join(f"[{s}]\n{o}" for s, o in failed))
    # No kernel may use scratch memory: a small array or struct indexed with
    # a register, or an argument block copied for such an access, costs every
    # launch (the large-M GEMM lost 20% to a 312-byte copy of its arguments).
    # SGPR spills go to VGPR lanes and are not scratch.
    with open(LIB_DIR / "resources.txt", "w") as f:
        for name in sorted(usage):
            u = usage[name]
            f.write(f"{name} vgprs={u.get('VGPRs', -1)} sgprs={u.get('TotalSGPRs', -1)} "
                    f"scratch={u.get('ScratchSize [bytes/lane]', -1)} occupancy={u.get('Occupancy [waves/SIMD]', -1)} "
                    f"lds={u.get('LDS Size [bytes/block]', -1)}\n")
    private = [n for n, u in usage.items() if u.get("ScratchSize [bytes/lane]", 0)]
    if private:
        raise RuntimeError("kernels using scratch memory:\n" + "\n".join(private[:20]))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)]
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    if res.returncode != 0:
        raise RuntimeError("HIP link failed:\n" + res.stdout.decode(errors="replace"))
    # every symbol must resolve now (a kernel whose host pass was dropped
    # leaves an undefined launch stub that only shows at load time)
    res = subprocess.run(["nm", "-D", "--undefined-only", str(tmp)], stdout=subprocess.PIPE)
    stubs = [ln for ln in res.stdout.decode().splitlines() if "device_stub" in ln]
    if stubs:
        raise RuntimeError("HIP link left undefined kernel stubs:\n" + "\n".join(stubs[:10]))
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
