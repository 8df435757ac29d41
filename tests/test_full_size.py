"""Parity at the benchmark configurations' full sizes.

* C1 (examples/linear.py MLP): 1000 SGD steps on the GPU against the CPU
  oracle, parameters within 1e-3 relative.
* C2 single-command benchmarks at their full shapes against float64 numpy
  (sampled rows for the 4096^3 product).
* C3 LayerNorm fwd+bwd [16384,1024] against the oracle, 3 SGD steps.
* C4 / C5 transformers (one training step at the real shapes): the oracle's
  naive kernels are too slow there, so the step is restated in float32
  torch on the CPU (the same math: per-head projections, per-sample
  attention scaled by 1/sqrt(d_model), softmax without max subtraction,
  post-norm LayerNorm with biased variance, ReLU FFN, MSE-to-zero loss, SGD
  lr 0.01) and every updated parameter is compared.
"""
import numpy as np
import pytest

import ad_amd as ad
from ad_amd import workloads
from oracle import OracleDevice

gpu = pytest.mark.gpu


def _rel_close(got, want, rel):
    for g, w in zip(got, want):
        scale = max(float(np.abs(w).max()), 1e-30)
        np.testing.assert_allclose(g, w, rtol=0, atol=rel * scale)


@gpu
def test_c1_mlp_1000_steps(hip):
    ad.reset()
    a = workloads.mlp(steps=1000)
    ad.execute(device=hip())
    ad.reset()
    b = workloads.mlp(steps=1000)
    ad.execute(device=OracleDevice())
    assert len(a["params"]) == len(b["params"]) == 4
    _rel_close(a["params"], b["params"], 1e-3)


@gpu
def test_c2_dotprod_elw_full(hip):
    """sigmoid(A@B + bias) on [4096,4096] x [4096,4096]: 64 sampled rows
    against float64, bounded by K * eps * |A| |B| before the sigmoid
    (slope <= 1/4)."""
    ad.reset()
    out = workloads.dotprod_elw(4096, 4096, 4096)
    ad.execute(device=hip())
    a, b, bias = out["inputs"]
    rows = np.random.default_rng(5).choice(4096, 64, replace=False)
    pre = a[rows].astype(np.float64) @ b.astype(np.float64) + bias
    want = 1.0 / (1.0 + np.exp(-pre))
    bound = 0.25 * 4 * 4096 * np.finfo(np.float32).eps * (np.abs(a[rows]) @ np.abs(b)).max() + 1e-6
    np.testing.assert_allclose(out["r"][rows], want, rtol=0, atol=bound)


@gpu
def test_c2_reduce_elw_full(hip):
    ad.reset()
    out = workloads.reduce_elw(8192, 4096, 0.5)
    ad.execute(device=hip())
    (x,) = out["inputs"]
    want = 0.5 * x.astype(np.float64).sum(-1)
    bound = 4096 * np.finfo(np.float32).eps * np.abs(x).sum(-1).max()
    np.testing.assert_allclose(out["r"], want, rtol=0, atol=bound)


@gpu
def test_c2_elw_chain_full(hip):
    ad.reset()
    out = workloads.elw_chain(64 << 20)
    ad.execute(device=hip())
    (x,) = out["inputs"]
    want = 3.0 / (np.exp2(x.astype(np.float64) * 0.5 + 1.0) + 1.0)
    np.testing.assert_allclose(out["r"], want, rtol=2e-6, atol=0)


@gpu
def test_c3_layernorm_full(hip):
    ad.reset()
    a = workloads.layernorm_train(16384, 1024, steps=3)
    ad.execute(device=hip())
    ad.reset()
    b = workloads.layernorm_train(16384, 1024, steps=3)
    ad.execute(device=OracleDevice())
    for x, y in zip(a["params"], b["params"]):
        np.testing.assert_allclose(x, y, rtol=1e-4, atol=1e-5)


def _torch_step(res, init, lr=0.01):
    """One training step of the traced encoder stack in float32 torch."""
    import torch
    torch.set_num_threads(max(1, min(16, torch.get_num_threads())))
    net = res["net"]
    t = {pid: torch.tensor(arr, requires_grad=True) for pid, arr in init.items()}
    x = torch.tensor(res["x"])

    def ln(h, m):
        mean = h.mean(-1, keepdim=True)
        var = ((h - mean) ** 2).mean(-1, keepdim=True)
        return (h - mean) / torch.sqrt(torch.abs(var + 1e-5)) * t[id(m.scale)] + t[id(m.bias)]

    out = x
    for layer in net:
        att = layer.attention
        heads = []
        for i in range(att.num_heads):
            q = out @ t[id(att.wq[i].w)]
            k = out @ t[id(att.wk[i].w)]
            v = out @ t[id(att.wv[i].w)]
            per = []
            for b in range(att.batch):
                rows = slice(b * att.seq, (b + 1) * att.seq)
                inner = (q[rows] @ k[rows].T) * (1.0 / np.sqrt(float(att.d_model)))
                e = torch.exp(inner)
                per.append((e / e.sum(-1, keepdim=True)) @ v[rows])
            heads.append(torch.cat(per, 0))
        y = torch.cat(heads, -1) @ t[id(att.wo.w)]
        y = ln(out + y, layer.layer_norm_att)
        ff = layer.ffwd
        h = torch.relu(y @ t[id(ff.f_expand.w)] + t[id(ff.f_expand.b)])
        z = h @ t[id(ff.f_contract.w)] + t[id(ff.f_contract.b)]
        out = ln(y + z, layer.layer_norm_ffwd)
    loss = (out * out * (1.0 / out.numel())).sum()
    loss.backward()
    with torch.no_grad():
        return {pid: (p - lr * p.grad).numpy() for pid, p in t.items()}


@gpu
@pytest.mark.parametrize("config,arena", [("c4", "packed"), ("c5", "packed"), ("c4", "unpacked"),
                                          ("c5", "unpacked")])
def test_transformer_step_full_size_vs_torch(hip, config, arena):
    layers, d, h, f, s, b = workloads.TRANSFORMER_CONFIGS[config]
    ad.reset()
    res = workloads.transformer(layers=layers, d_model=d, heads=h, ff=f, seq=s, batch=b, steps=1,
                                receive=False)
    init = {id(p): p.arr.copy() for p in res["params_ref"]}
    ad.execute(device=hip(arena=arena))
    want = _torch_step(res, init)
    for p in res["params_ref"]:
        np.testing.assert_allclose(p.arr, want[id(p)], rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("shape", [(2, 32, 4, 64, 8, 2), (1, 16, 2, 32, 4, 4)])
def test_torch_reference_matches_oracle(shape):
    """The torch restatement of the training step used above agrees with the
    CPU oracle on small encoder stacks (so it restates the same graph).
    Every reduction length here is a power of two, as at C4/C5: for other
    lengths the reference's work-group tree drops elements (reduce.py:38-43)
    and a plain sum no longer restates it."""
    layers, d, h, f, s, b = shape
    ad.reset()
    res = workloads.transformer(layers=layers, d_model=d, heads=h, ff=f, seq=s, batch=b, steps=1,
                                receive=False)
    init = {id(p): p.arr.copy() for p in res["params_ref"]}
    ad.execute(device=OracleDevice())
    want = _torch_step(res, init)
    for p in res["params_ref"]:
        np.testing.assert_allclose(p.arr, want[id(p)], rtol=1e-4, atol=1e-6)

