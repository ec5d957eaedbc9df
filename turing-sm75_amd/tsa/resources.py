"""Per-kernel resource usage of the gfx950 build: VGPRs, AGPRs, scratch (spill) bytes per lane,
occupancy (waves per SIMD) and LDS bytes per workgroup, read from the compiler's
kernel-resource-usage remarks.  The counterpart of the reference's ptxas report, which its
Makefile asks for on every kernel build (-Xptxas=-v, Makefile:21,25).

    python3 tsa/resources.py [--hipcc PATH] [--out FILE] csrc/a.hip csrc/b.hip ...

compiles each file for the device only (no object is kept) with the library's own flags plus
-Rpass-analysis=kernel-resource-usage and writes one line per kernel.  The Makefile runs it
beside the library build (lib/resource-usage.txt); tests/test_resource_usage.py checks the
hot kernels' lines against their stated budgets.
"""
from __future__ import annotations

import argparse
import os
import re
import shutil
import subprocess
import sys

ARCH = "gfx950"
# the library's device flags (turing-sm75_amd/Makefile, HIPFLAGS), without -fPIC / -Wall
FLAGS = ["--offload-arch=" + ARCH, "-O3", "-std=c++17",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
_FIELDS = {"VGPRs": "vgpr", "AGPRs": "agpr", "ScratchSize [bytes/lane]": "scratch",
           "Occupancy [waves/SIMD]": "occupancy", "LDS Size [bytes/block]": "lds",
           "VGPRs Spill": "vgpr_spill", "SGPRs Spill": "sgpr_spill"}
_REMARK = re.compile(r"remark:\s+(Function Name|[A-Za-z][A-Za-z /\[\]]*?):\s+(\S+)\s+\[-Rpass-analysis")


def _hipcc(path: str | None) -> str:
    return path or os.environ.get("HIPCC") or "/opt/rocm/bin/hipcc"


def kernels(files, hipcc: str | None = None) -> dict[str, dict[str, int]]:
    """{mangled kernel name: {vgpr, agpr, scratch, occupancy, lds, vgpr_spill, sgpr_spill}} over
    the given .hip sources (raises CalledProcessError when a file does not compile)."""
    out: dict[str, dict[str, int]] = {}
    for f in files:
        r = subprocess.run([_hipcc(hipcc), *FLAGS, "--cuda-device-only", "-c", "-x", "hip", f,
                            "-o", os.devnull, "-Rpass-analysis=kernel-resource-usage"],
                           capture_output=True, text=True)
        if r.returncode != 0:
            sys.stderr.write("\n".join(l for l in r.stderr.splitlines() if "remark:" not in l) + "\n")
            r.check_returncode()
        cur = None
        for line in r.stderr.splitlines():
            m = _REMARK.search(line)
            if not m:
                continue
            key, val = m.group(1).strip(), m.group(2)
            if key == "Function Name":
                cur = out.setdefault(val, {})
            elif cur is not None and key in _FIELDS:
                cur[_FIELDS[key]] = int(val) if val.isdigit() else 0
    return out


def demangle(names) -> dict[str, str]:
    """Readable names (c++filt when it is installed; the mangled name otherwise)."""
    names = list(names)
    tool = shutil.which("c++filt")
    if not tool or not names:
        return {n: n for n in names}
    # this c++filt does not know _Float16 (DF16_); for display it is written as half (Dh)
    r = subprocess.run([tool], input="\n".join(n.replace("DF16_", "Dh") for n in names),
                       capture_output=True, text=True)
    lines = r.stdout.splitlines()
    return dict(zip(names, lines)) if len(lines) == len(names) else {n: n for n in names}


def table(res: dict[str, dict[str, int]]) -> str:
    pretty = demangle(res)
    rows = ["vgpr agpr scratch occupancy lds  kernel"]
    for n in sorted(res, key=lambda n: pretty[n]):
        r = res[n]
        rows.append(f"{r.get('vgpr', 0):4d} {r.get('agpr', 0):4d} {r.get('scratch', 0):7d} "
                    f"{r.get('occupancy', 0):9d} {r.get('lds', 0):6d}  {pretty[n]}")
    return "\n".join(rows) + "\n"


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--hipcc")
    ap.add_argument("--out")
    ap.add_argument("files", nargs="+")
    a = ap.parse_args(argv)
    text = table(kernels(a.files, a.hipcc))
    if a.out:
        tmp = a.out + ".tmp"
        with open(tmp, "w") as fh:
            fh.write(text)
        os.replace(tmp, a.out)
    else:
        sys.stdout.write(text)
    return 0


if __name__ == "__main__":
    sys.exit(main())
