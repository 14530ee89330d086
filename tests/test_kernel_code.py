"""CPU checks of the generated gfx950 code of the MFMA tile engine.

The GEMM kernels hold 256 fp32 accumulators per lane in AGPRs and run close to the
256-VGPR limit.  A small source change can tip the register allocator into moving
values between VGPRs and AGPRs (v_accvgpr_read / v_accvgpr_write) or into scratch
inside the K loop, which costs 20-30 % of the kernel's time without changing any
result; a range check on permutation entries once did exactly that to the MoE
gate/up pass.  This test compiles cdx_gemm.hip to assembly (hipcc, no GPU needed)
and checks that the K loop of every engine instantiation is free of both (the 128 x 128
tiles of small products: at most a bounded number of accumulator copies, see below) and
holds the expected MFMA count per iteration (two K32 sub-steps of 8 x 8 blocks per wave for
256 x 256 tiles, of (BM / 32) x (BN / 32) blocks for the narrower tiles of small
products).  The
persistent form (gemm_persist_kernel) nests its K loop inside the loop over tiles; its
K-loop block (the one issuing a whole step's 128 MFMAs and 16 DMAs) gets the same
checks, and the kernel as a whole must not touch scratch memory.
"""

from __future__ import annotations

import re
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
HIPCC = "/opt/rocm/bin/hipcc"


@pytest.fixture(scope="module")
def gemm_asm(tmp_path_factory):
    if not Path(HIPCC).exists():
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("asm") / "cdx_gemm.s"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "--cuda-device-only", "-S", str(REPO / "complexity-deep_amd/csrc/cdx_gemm.hip"),
           "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True)
    return out.read_text()


def _main_loops(asm: str):
    for name in re.findall(r"^(_ZN3cdx14gemm_nt_kernel\S+):", asm, re.M):
        start = asm.index(name + ":")
        body = asm[start:asm.index(".Lfunc_end", start)]
        loops = [m.group(1) for m in re.finditer(r"^\.LBB\d+_\d+:[^\n]*Loop Header[^\n]*\n(.*?)(?=^\.LBB|\Z)",
                                                 body, re.M | re.S) if "v_mfma" in m.group(1)]
        yield name, loops


def test_gemm_k_loops_have_no_register_shuffles(gemm_asm):
    seen = 0
    for name, loops in _main_loops(gemm_asm):
        assert len(loops) == 1, f"{name}: expected one MFMA loop, found {len(loops)}"
        loop = loops[0]
        seen += 1
        cfg = [int(v) for v in re.search(r"GemmCfgI((?:Li\d+E)+)", name).group(1)[2:-1].split("ELi")]
        bn, bm = cfg[0], (cfg[7] if len(cfg) > 7 else 256)
        # two K32 sub-steps of (BM/32) x (BN/32) blocks of 16 x 16 per wave
        assert loop.count("v_mfma_f32_16x16x32_bf16") == 2 * (bm // 32) * (bn // 32), name
        if (bm, bn) == (128, 128):
            # The 128 x 128 tiles of small products keep three LDS stages, and with them
            # the register allocator copies some of the 64 accumulator registers per K
            # step for some epilogues; measured, three stages with the copies beat two
            # without them.  Bound the copies so that a change that makes it worse fails.
            n = loop.count("v_accvgpr_read") + loop.count("v_accvgpr_write") + loop.count("v_accvgpr_mov")
            assert n <= 96, f"{name}: {n} accumulator copies per K step"
        else:
            assert "v_accvgpr_read" not in loop and "v_accvgpr_write" not in loop, \
                f"{name}: VGPR/AGPR shuffles inside the K loop"
        assert "scratch_" not in loop and "buffer_store" not in loop, f"{name}: spills inside the K loop"
    assert seen >= 10


def _blocks(body: str):
    parts = re.split(r"^(\.LBB\d+_\d+):", body, flags=re.M)
    yield "entry", parts[0]
    for i in range(1, len(parts), 2):
        yield parts[i], parts[i + 1]


def test_persistent_gemm_k_loops_have_no_register_shuffles(gemm_asm):
    seen = 0
    for name in re.findall(r"^(_ZN3cdx19gemm_persist_kernel\S+):", gemm_asm, re.M):
        start = gemm_asm.index(name + ":")
        body = gemm_asm[start:gemm_asm.index(".Lfunc_end", start)]
        assert "scratch_" not in body, f"{name}: scratch memory in use"
        # The K-loop block branches back to itself (a tile's last step, which can also
        # carry 16 DMAs, falls through into the epilogue instead).
        k_loops = [txt for label, txt in _blocks(body)
                   if txt.count("v_mfma_f32_16x16x32_bf16") == 128 and txt.count(" lds") == 16
                   and re.search(r"s_cbranch_\w+ " + re.escape(label) + r"\b", txt)]
        assert k_loops, f"{name}: no K-loop block with 128 MFMAs and 16 DMAs"
        for loop in k_loops:
            assert "v_accvgpr_read" not in loop and "v_accvgpr_write" not in loop, \
                f"{name}: VGPR/AGPR shuffles inside the K loop"
        seen += 1
    assert seen >= 3
