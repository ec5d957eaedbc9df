"""Register, scratch, occupancy and LDS budgets of the hot kernels, from the compiler's
kernel-resource-usage remarks (the counterpart of the reference's -Xptxas=-v on every build,
Makefile:21,25).  The sources are compiled here for the device only (no GPU needed); a kernel
that starts to spill, or whose registers or LDS no longer let the stated number of waves
share a SIMD, fails the suite instead of showing up only as a slower bench.

Budgets (per kernel: registers = VGPRs + AGPRs of one wave; waves per SIMD; LDS per workgroup):
  attn_fwd_kernel<64>           4 waves / SIMD,  32 KiB LDS (4-wave workgroups of 128 rows)
  attn_fwd_kernel<128>          2 waves / SIMD,  64 KiB LDS
  attn_fwd_kernel<256>          2 waves / SIMD, 128 KiB LDS (8-wave workgroups, one per CU)
  gdn_chunk_prep (fp16 I/O)     4 workgroups / CU: 128 registers, 40 KiB LDS
  gdn_chunk_prep (fp32 I/O)     3 workgroups / CU (the V_lo tile: 53.25 KiB of LDS)
  gdn_chunk_carry               one 8-wave workgroup per CU: 2 waves / SIMD, up to 160 KiB LDS
  gdn_decode_kernel, gdn_recurrent_kernel, the pre/post-op passes: 8 waves / SIMD
  and no kernel on the product path spills (scratch 0).  The naive check kernels are exempt
  from the spill rule: they are the drivers' correctness references, not hot paths.
"""
import os
import re
import shutil

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "turing-sm75_amd")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

pytestmark = pytest.mark.skipif(not os.path.exists(HIPCC) and not shutil.which("hipcc"),
                                reason="hipcc not installed")

# (pattern on the mangled name, min waves per SIMD, max registers, max LDS bytes)
BUDGETS = [
    (r"attn_fwd_kernelILi64E", 4, 128, 32 << 10),
    (r"attn_fwd_kernelILi128E", 2, 256, 64 << 10),
    (r"attn_fwd_kernelILi256E", 2, 256, 128 << 10),
    (r"gdn_chunk_prepILb[01]EDF16_E", 4, 128, 40 << 10),
    (r"gdn_chunk_prepILb0EfE", 3, 168, (160 << 10) // 3),
    (r"gdn_chunk_carry", 2, 256, 160 << 10),
    (r"gdn_decode_kernel", 8, 64, 4 << 10),
    (r"gdn_recurrent_kernel", 8, 64, 4 << 10),
    (r"gated_rmsnorm_kernel", 8, 64, 0),
    (r"l2norm_rows_kernel", 8, 64, 0),
    (r"gdn_gates_kernel", 8, 64, 0),
]
CHECK_KERNELS = re.compile(r"attn_naive_kernel|gdn_naive_kernel")


@pytest.fixture(scope="module")
def usage():
    import sys
    sys.path.insert(0, PKG)
    from tsa import resources
    mk = open(os.path.join(PKG, "Makefile")).read()
    hip = re.search(r"^HIPSRC := (.*)$", mk, re.M).group(1).split()
    assert hip and all(f.endswith(".hip") for f in hip)
    cwd = os.getcwd()
    os.chdir(PKG)
    try:
        res = resources.kernels(hip, HIPCC if os.path.exists(HIPCC) else shutil.which("hipcc"))
    finally:
        os.chdir(cwd)
    print(resources.table(res))
    return res


@pytest.mark.parametrize("pattern,waves,regs,lds", BUDGETS, ids=[b[0] for b in BUDGETS])
def test_hot_kernel_budget(usage, pattern, waves, regs, lds):
    hits = {n: r for n, r in usage.items() if re.search(pattern, n)}
    assert hits, f"no kernel matches {pattern}"
    for n, r in hits.items():
        assert r["scratch"] == 0 and r.get("vgpr_spill", 0) == 0, (n, r)
        assert r["occupancy"] >= waves, (n, r)
        assert r["vgpr"] + r["agpr"] <= regs, (n, r)
        assert r["lds"] <= lds, (n, r)


def test_no_product_kernel_spills(usage):
    spills = {n: r["scratch"] for n, r in usage.items() if r["scratch"] and not CHECK_KERNELS.search(n)}
    assert not spills, spills


def test_report_covers_every_kernel(usage):
    # every __global__ of the library reports; the Makefile writes the same table to
    # lib/resource-usage.txt on each build
    assert len(usage) >= 40, sorted(usage)
    for r in usage.values():
        assert {"vgpr", "agpr", "scratch", "occupancy", "lds"} <= set(r), r
