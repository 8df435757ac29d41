"""DotProd kernels computed on the host in lockstep (every thread of a block
a fiber of its own, real barriers, the MFMAs and cross-lane shuffles
emulated with the hardware's lane layout; ``host_emulation.LOCKSTEP_SHIM``)
against float64 numpy: the MFMA tile kernels (64 x 64 and 128 x 128 tiles,
split K with its combine pass), ``dp_quad`` for small launch groups, the
skinny and direct kernels, transposed operands and fused epilogues, and the
bf16 option's kernel -- the GPU path's own generated code, checked before any
GPU run."""
import numpy as np
import pytest

import ad_amd as ad
from ad_amd.graph import Receiver, Tensor

from .host_emulation import host_arena


def _run(tmp_path, M, K, N, ta, tb, epilogue, **options):
    rng = np.random.default_rng(M * 7 + K * 3 + N + 2 * ta + tb)
    a = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    b = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    bias = rng.standard_normal((N,)).astype(np.float32)
    ad.reset()
    A, B = Tensor(a), Tensor(b)
    r = (A.T() if ta else A) @ (B.T() if tb else B)
    outs = [r + Tensor(bias), (r + Tensor(bias)).sigmoid()] if epilogue else [r]
    Receiver(lambda *v: None, outs)
    dev, arena = host_arena(ad.compile_proc(), str(tmp_path), lockstep=True, **options)
    assert arena is not None, "a launch left the arena or a barrier timed out"
    vals = [arena[off:off + nb].view(np.float32).reshape(M, N) for off, nb in dev.ctx.reads[:len(outs)]]
    a64 = (a.T if ta else a).astype(np.float64)
    b64 = (b.T if tb else b).astype(np.float64)
    ref = a64 @ b64 + (bias if epilogue else 0.0)
    eps = np.finfo(np.float32).eps
    bound = np.sqrt(K) * eps * (np.abs(a64) @ np.abs(b64)) + 4 * eps * np.abs(bias if epilogue else 0.0) + 1e-7
    err = np.abs(vals[0] - ref)
    assert np.all(err <= bound), f"{np.max(err / bound):.2f} x the bound"
    if epilogue:
        np.testing.assert_allclose(vals[1], 1 / (1 + np.exp(-vals[0].astype(np.float64))), rtol=1e-5, atol=1e-6)
    plans = [p for ps in dev.kernels.values() for p in ps] + list(getattr(dev, "_narrow_plans", {}).values())
    return " ".join(p.source for p in plans)


@pytest.mark.parametrize("M,K,N,ta,tb,epilogue,kernel", [
    (64, 64, 64, False, False, False, "dp_mfma<64, 64, 1, 64"),
    (130, 70, 257, True, False, True, "dp_mfma<64, 64, 1, 64"),
    (96, 200, 100, False, True, True, "dp_mfma<64, 64, 1, 64"),
    (520, 136, 520, True, True, True, "dp_mfma<128, 128, 1, 32"),
    (2, 255, 255, False, False, True, "dp_skinny<8>"),
    (100, 2, 130, False, True, False, "dp_direct"),
])
def test_tile_kernels_on_host(tmp_path, M, K, N, ta, tb, epilogue, kernel):
    """The MFMA tile kernel at both tile sizes (ragged M, N and K,
    transposed operands, float4 and per-element epilogues), and the
    skinny and direct kernels, with narrow launches off."""
    src = _run(tmp_path, M, K, N, ta, tb, epilogue, narrow_launches=False)
    assert kernel in src


@pytest.mark.parametrize("M,K,N,ta,tb,epilogue,kernel", [
    (256, 512, 64, False, False, True, "dp_quad<1, 128>"),   # one 128-deep panel per wave and round, 4 rounds
    (130, 300, 257, True, True, True, "dp_quad<1, 128>"),    # ragged K: a partial last panel
    (64, 1024, 64, False, True, False, "dp_quad<4, 128>"),   # K split in 4 chunks of 256, then the combine pass
    (512, 64, 100, True, False, True, "dp_quad<1, 64>"),     # K = 64: 64-deep panels
])
def test_quad_kernel_on_host(tmp_path, M, K, N, ta, tb, epilogue, kernel):
    """dp_quad, the kernel of launch groups too small to fill the device
    (32 x 32 tiles, each block's K panels split among its four waves, the
    partial tiles added through LDS)."""
    src = _run(tmp_path, M, K, N, ta, tb, epilogue)
    assert kernel in src


def _bf16(x):
    """float32 -> bfloat16 (round to nearest even) -> float64."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32).astype(np.float64)


@pytest.mark.parametrize("M,K,N,ta,tb", [(64, 64, 64, False, False), (130, 70, 257, True, True),
                                         (96, 200, 100, False, True)])
def test_bf16_kernel_on_host(tmp_path, M, K, N, ta, tb):
    """The bf16 DotProd option (operands packed to k-contiguous bfloat16,
    v_mfma_f32_32x32x16_bf16, fp32 sums) against float64 products of the
    same bfloat16-rounded operands: only the fp32 summation differs, so
    the bound is K eps (|A| @ |B|) -- far tighter than the rounding of the
    operands themselves, which the check also sees."""
    rng = np.random.default_rng(M * 13 + K * 5 + N)
    a = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    b = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    bias = rng.standard_normal((N,)).astype(np.float32)
    ad.reset()
    r = ((Tensor(a).T() if ta else Tensor(a)) @ (Tensor(b).T() if tb else Tensor(b))) + Tensor(bias)
    Receiver(lambda v: None, [r])
    dev, arena = host_arena(ad.compile_proc(), str(tmp_path), lockstep=True, dot_precision="bf16", bf16_min_macs=0)
    assert arena is not None, "a launch left the arena or a barrier timed out"
    assert any("dp_bf16<" in p.source for ps in dev.kernels.values() for p in ps)
    off, nb = dev.ctx.reads[0]
    got = arena[off:off + nb].view(np.float32).reshape(M, N)
    a64, b64 = (_bf16(a).T if ta else _bf16(a)), (_bf16(b).T if tb else _bf16(b))
    ref = a64 @ b64 + bias
    bound = (K + 2) * np.finfo(np.float32).eps * (np.abs(a64) @ np.abs(b64) + np.abs(bias)) + 1e-7
    err = np.abs(got - ref)
    assert np.all(err <= bound), f"{np.max(err / bound):.2f} x the bound"
    exact = (a.T if ta else a).astype(np.float64) @ (b.T if tb else b).astype(np.float64) + bias
    assert np.max(np.abs(got - exact)) > 10 * np.max(bound), "the operands were not rounded to bfloat16"
