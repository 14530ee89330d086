"""CPU checks of the C-ABI boundary (no kernel is launched).

* libcdx.so loads and exports every function declared in include/cdx.h, and the
  ctypes table in complexity_deep/_native.py binds exactly that set.
* Host-side argument validation rejects bad calls with the documented status codes
  and a message, before anything is enqueued (so these run without a GPU).
* The product fails loudly instead of falling back: CPU tensors and a missing
  library raise.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

REPO = Path(__file__).resolve().parents[1]
HEADER = REPO / "include" / "cdx.h"

CDX_EINVAL, CDX_EUNSUPPORTED, CDX_EWORKSPACE = -1, -2, -4


def _declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(cdx_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from complexity_deep import _native
    if not _native.LIB_PATH.exists():
        import importlib.util
        spec = importlib.util.spec_from_file_location("build_native", REPO / "complexity-deep_amd" / "build_native.py")
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build()
    return _native.lib()


def test_header_symbols_exported(lib):
    from complexity_deep import _native
    names = _declared()
    assert len(names) >= 10
    for n in names:
        assert hasattr(lib, n), f"{n} declared in cdx.h but not exported"
    assert sorted(_native.exported_symbols()) == names


def test_version_and_error_string(lib):
    assert lib.cdx_version() >= 100
    assert isinstance(lib.cdx_last_error(), bytes)


def test_norm_validation(lib):
    rc = lib.cdx_add_rmsnorm_fwd(16, None, 16, 1e-6, 4, 7, 16, None, None)
    assert rc == CDX_EUNSUPPORTED and b"multiple of 8" in lib.cdx_last_error()
    assert lib.cdx_add_rmsnorm_fwd(16, None, 16, 1e-6, -1, 8, 16, None, None) == CDX_EINVAL
    assert lib.cdx_add_rmsnorm_fwd(None, None, None, 1e-6, 4, 8, None, None, None) == CDX_EINVAL
    assert lib.cdx_add_rmsnorm_fwd(16, None, 16, -1.0, 4, 8, 16, None, None) == CDX_EINVAL
    assert lib.cdx_add_rmsnorm_fwd(16, None, 16, 1e-6, 4, 8, 16, 32, None) == CDX_EINVAL  # residual_out w/o residual
    assert lib.cdx_add_rmsnorm_fwd(18, None, 16, 1e-6, 4, 8, 16, None, None) == CDX_EUNSUPPORTED  # misaligned
    assert lib.cdx_add_rmsnorm_fwd(None, None, None, 1e-6, 0, 8, None, None, None) == 0  # T == 0 is a no-op
    # the strided-output plain norm: (x, weight, eps, T, H, out, ldo)
    assert lib.cdx_rmsnorm_ld_fwd(16, 16, 1e-6, 4, 64, 16, 32, None) == CDX_EINVAL  # ldo < H
    assert lib.cdx_rmsnorm_ld_fwd(16, 16, 1e-6, 4, 64, 16, 132, None) == CDX_EUNSUPPORTED  # ldo % 8
    assert lib.cdx_rmsnorm_ld_fwd(16, 16, 1e-6, 4, 60, 16, 128, None) == CDX_EUNSUPPORTED  # H % 8
    assert lib.cdx_rmsnorm_ld_fwd(16, 16, -1.0, 4, 64, 16, 128, None) == CDX_EINVAL  # eps
    assert lib.cdx_rmsnorm_ld_fwd(None, 16, 1e-6, 4, 64, 16, 128, None) == CDX_EINVAL
    assert lib.cdx_rmsnorm_ld_fwd(16, 16, 1e-6, 4, 64, 24, 128, None) == CDX_EUNSUPPORTED  # misaligned out
    assert b"cdx_rmsnorm_ld_fwd" in lib.cdx_last_error()
    assert lib.cdx_rmsnorm_ld_fwd(None, None, 1e-6, 0, 64, None, 128, None) == 0  # T == 0


def test_route_validation(lib):
    # One int32 per (block, expert); blocks of 1024 tokens, at most 256 blocks.
    assert lib.cdx_route_workspace_bytes(0, 4) == 0
    assert lib.cdx_route_workspace_bytes(1024, 4) == 1 * 4 * 4
    assert lib.cdx_route_workspace_bytes(1025, 8) == 2 * 8 * 4
    assert lib.cdx_route_workspace_bytes(256 * 1024, 64) == 256 * 64 * 4
    assert lib.cdx_route_workspace_bytes(256 * 1024 + 1, 64) == 129 * 64 * 4  # blocks of 2048 tokens
    assert lib.cdx_route_workspace_bytes(2 ** 31 - 1, 64) == 256 * 64 * 4
    assert lib.cdx_route_plan(16, 10, 16, 5, 65, 16, 16, 16, 16, 16, 16, 1 << 20, None) == CDX_EUNSUPPORTED
    assert lib.cdx_route_plan(16, 10, 16, 0, 4, 16, 16, 16, 16, 16, 16, 1 << 20, None) == CDX_EINVAL
    assert lib.cdx_route_plan(16, 2048, 16, 5, 4, 16, 16, 16, 16, 16, 16, 8, None) == CDX_EWORKSPACE
    assert lib.cdx_route_plan(16, -1, 16, 5, 4, 16, 16, 16, 16, 16, 16, 0, None) == CDX_EINVAL
    assert lib.cdx_route_plan(None, 10, 16, 5, 4, 16, 16, 16, 16, 16, 16, 1 << 20, None) == CDX_EINVAL
    assert lib.cdx_permute_rows(16, 16, 1 << 31, 24, 16, None) == CDX_EUNSUPPORTED  # T >= 2^31
    assert lib.cdx_permute_rows(16, 16, 4, 0, 16, None) == CDX_EINVAL
    assert lib.cdx_permute_rows(None, 16, 4, 6, 16, None) == CDX_EINVAL
    assert lib.cdx_unpermute_rows(None, None, 0, 32, None, None) == 0


def test_hbm_probe_validation(lib):
    assert lib.cdx_hbm_probe(3, 16, 16, 1024, None) == CDX_EINVAL
    assert lib.cdx_hbm_probe(0, 16, 16, 1000, None) == CDX_EINVAL  # not a multiple of 16
    assert lib.cdx_hbm_probe(2, None, 16, 1024, None) == CDX_EINVAL
    assert lib.cdx_hbm_probe(0, 8, 16, 1024, None) == CDX_EUNSUPPORTED  # misaligned
    assert lib.cdx_hbm_probe(1, None, None, 0, None) == 0


def test_route_plans_validation(lib):
    # One count table per plan.
    assert lib.cdx_route_plans_workspace_bytes(1025, 8, 24) == 24 * 2 * 8 * 4
    assert lib.cdx_route_plans_workspace_bytes(1025, 8, 0) == 0
    maps = (ctypes.c_void_p * 2)(16, 16)
    table = ctypes.cast(maps, ctypes.c_void_p)
    assert lib.cdx_route_plans(16, 10, table, -1, 5, 4, 16, 16, 16, 16, 16, 16, 1 << 20, None) == CDX_EINVAL
    assert lib.cdx_route_plans(16, 10, table, 0, 5, 4, 16, 16, 16, 16, 16, 16, 1 << 20, None) == 0  # no plans
    assert lib.cdx_route_plans(16, 10, None, 2, 5, 4, 16, 16, 16, 16, 16, 16, 1 << 20, None) == CDX_EINVAL
    nulls = ctypes.cast((ctypes.c_void_p * 2)(16, None), ctypes.c_void_p)
    assert lib.cdx_route_plans(16, 10, nulls, 2, 5, 4, 16, 16, 16, 16, 16, 16, 1 << 20, None) == CDX_EINVAL
    assert b"map 1 is NULL" in lib.cdx_last_error()
    assert lib.cdx_route_plans(16, 10, table, 2, 5, 65, 16, 16, 16, 16, 16, 16, 1 << 20, None) == CDX_EUNSUPPORTED
    assert lib.cdx_route_plans(16, 2048, table, 2, 5, 4, 16, 16, 16, 16, 16, 16, 16, None) == CDX_EWORKSPACE
    assert lib.cdx_route_plans(16, 1 << 30, table, 2, 5, 4, 16, 16, 16, 16, 16, 16, 1 << 30, None) == \
        CDX_EUNSUPPORTED  # L * T >= 2^31


def test_gemm_validation(lib):
    assert lib.cdx_mu_qkv_fwd(16, 96, 16, 96, 16, 16, 192, 8, 96, 64, 16, 64, None) == CDX_EUNSUPPORTED  # H % 64
    assert lib.cdx_mu_qkv_fwd(16, 64, 16, 64, 16, 16, 128, 8, 64, 60, 16, 64, None) == CDX_EUNSUPPORTED  # N % 8
    assert lib.cdx_mu_qkv_fwd(16, 32, 16, 64, 16, 16, 128, 8, 64, 64, 16, 64, None) == CDX_EINVAL  # ldx < H
    assert lib.cdx_mu_qkv_fwd(16, 64, 16, 64, 16, 16, 32, 8, 64, 64, 16, 64, None) == CDX_EINVAL  # ldw < H
    assert lib.cdx_mu_qkv_fwd(16, 64, 16, 64, 16, None, 64, 8, 64, 64, 16, 64, None) == CDX_EINVAL  # mu w/o w_mu
    assert lib.cdx_moe_swiglu_fwd(16, 8, 96, 64, 4, 1, 16, 16, 16, 16, 16, 16, None) == CDX_EUNSUPPORTED
    assert lib.cdx_moe_swiglu_fwd(16, 8, 64, 64, 65, 1, 16, 16, 16, 16, 16, 16, None) == CDX_EINVAL
    assert lib.cdx_moe_swiglu_fwd(None, 0, 64, 64, 4, 1, None, None, None, None, None, None, None) == 0
    assert lib.cdx_grouped_gemm_fwd(16, 8, 48, 64, 4, 16, 16, 16, None) == CDX_EUNSUPPORTED
    assert b"multiple of 64" in lib.cdx_last_error()
    # gate/up operand beyond 4 GB: (64 + 1) * 2 * 8192 * 8192 * 2 bytes
    assert lib.cdx_moe_swiglu_fwd(16, 8, 8192, 8192, 64, 1, 16, 16, 16, 16, 16, 16, None) == CDX_EUNSUPPORTED
    assert lib.cdx_mu_guidance_fwd(16, 8, 64, 16, 16, 2.0, 0.0, -2.0, 2.0, 16, 64, None) == CDX_EINVAL  # mu_lo > mu_hi
    assert lib.cdx_mu_guidance_fwd(16, 8, 64, 16, None, 0.0, 2.0, -2.0, 2.0, 16, 64, None) == CDX_EINVAL  # no mu
    assert lib.cdx_mu_guidance_fwd(16, 8, 64, 16, 16, 0.0, 2.0, -2.0, 2.0, 16, 32, None) == CDX_EINVAL  # ldo < H
    assert lib.cdx_mu_guidance_fwd(16, 8, 64, 16, 16, 0.0, 2.0, -2.0, 2.0, 16, 68, None) == CDX_EUNSUPPORTED  # ldo % 8
    assert lib.cdx_mu_guidance_fwd(None, 0, 64, None, None, 0.0, 2.0, -2.0, 2.0, None, 128, None) == 0  # T = 0
    assert lib.cdx_linear_fwd(16, 64, 16, 64, 8, 64, 30, 16, 30, None) == CDX_EINVAL  # ldo < round_up(N, 8)
    assert lib.cdx_linear_residual_fwd(16, 64, 16, 64, 8, 64, 30, 16, 32, None) == CDX_EUNSUPPORTED  # N % 8
    assert lib.cdx_linear_residual_fwd(16, 96, 16, 96, 8, 96, 32, 16, 32, None) == CDX_EUNSUPPORTED  # K % 64
    assert lib.cdx_linear_residual_fwd(16, 64, 16, 64, 8, 64, 32, 16, 16, None) == CDX_EINVAL  # ldr < N
    assert lib.cdx_linear_residual_fwd(16, 64, 16, 64, 1 << 31, 64, 32, 16, 32, None) == CDX_EUNSUPPORTED  # M
    assert lib.cdx_linear_residual_fwd(None, 64, None, 64, 0, 64, 32, None, 32, None) == 0  # M = 0


def test_qkv_rope_validation(lib):
    # (x, ldx, mu, ldmu, w, w_mu, ldw, B, S, H, nq, nkv, hd, qn, kn, eps, cos_sin, n_pos, pos0, q, k, v, vt_ld)
    ok = [16, 128, 16, 128, 16, 16, 128, 1, 4, 128, 2, 1, 64, None, None, 1e-6, 16, 4, 0, 16, 16, 16, 0]

    def rope(**kw):
        args = list(ok)
        names = ["x", "ldx", "mu", "ldmu", "w", "w_mu", "ldw", "B", "S", "H", "nq", "nkv", "hd", "qn", "kn", "eps",
                 "cos_sin", "n_pos", "pos0", "q", "k", "v", "vt_ld"]
        for key, val in kw.items():
            args[names.index(key)] = val
        return lib.cdx_mu_qkv_rope_fwd(*args, None)

    assert rope(hd=48, B=0) == CDX_EUNSUPPORTED
    assert rope(ldmu=64, B=0) == CDX_EINVAL                      # mu rows shorter than H
    assert rope(qn=16, B=0) == CDX_EINVAL                        # one QK norm weight only
    assert rope(vt_ld=65, B=0) == CDX_EINVAL
    assert rope(n_pos=3) == CDX_EINVAL                           # table shorter than pos0 + S
    assert rope(w_mu=None) == CDX_EINVAL                         # mu without its weights
    assert rope(B=0) == 0                                        # no rows: nothing to do

    # (x, ldx, mu_row, w, w_mu, ldw, B, S, H, nq, nkv, hd, qn, kn, eps, cos_sin, n_pos, pos0, q, k, v, vt_ld, work)
    bc = [16, 128, 16, 16, 16, 128, 1, 4, 128, 2, 1, 64, None, None, 1e-6, 16, 4, 0, 16, 16, 16, 0, 16]

    def bcast(**kw):
        args = list(bc)
        names = ["x", "ldx", "mu_row", "w", "w_mu", "ldw", "B", "S", "H", "nq", "nkv", "hd", "qn", "kn", "eps",
                 "cos_sin", "n_pos", "pos0", "q", "k", "v", "vt_ld", "work"]
        for key, val in kw.items():
            args[names.index(key)] = val
        return lib.cdx_mu_qkv_rope_bcast_fwd(*args, None)

    assert bcast(mu_row=None) == CDX_EINVAL
    assert bcast(work=None) == CDX_EINVAL                        # the fold needs its scratch
    assert bcast(work=24) == CDX_EUNSUPPORTED                    # scratch not 16-byte aligned
    assert bcast(ldw=132) == CDX_EUNSUPPORTED                    # B stride not a multiple of 8
    assert bcast(w_mu=None) == CDX_EINVAL
    assert bcast(H=96) == CDX_EUNSUPPORTED
    assert b"cdx_mu_qkv_rope_bcast_fwd" in lib.cdx_last_error()
    assert bcast(B=0, work=None) == 0                            # no rows: nothing to do


def test_cpu_tensors_raise():
    from complexity_deep.normalization import add_rms_norm
    x = torch.randn(4, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        add_rms_norm(x, None, torch.ones(64, dtype=torch.bfloat16))


def test_missing_library_raises(monkeypatch, tmp_path):
    from complexity_deep import _native
    monkeypatch.setattr(_native, "_lib", None)
    monkeypatch.setattr(_native, "LIB_PATH", tmp_path / "libcdx.so")
    with pytest.raises(_native.NativeLibraryMissing):
        _native.lib()


def test_forward_only_guard():
    from complexity_deep import ComplexityConfig, ComplexityModel
    cfg = ComplexityConfig(vocab_size=64, hidden_size=64, intermediate_size=128, num_hidden_layers=1,
                           num_attention_heads=2, num_key_value_heads=1)
    m = ComplexityModel(cfg)
    with pytest.raises(NotImplementedError, match="forward-only"):
        m(torch.zeros(1, 4, dtype=torch.long))


def test_ctypes_only_plain_types():
    from complexity_deep import _native
    for name, (res, args) in _native._SIGNATURES.items():
        for a in args:
            assert a in (ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_float, ctypes.c_size_t), name
