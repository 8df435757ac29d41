"""Float32 torch restatement of the encoder training step that
``ad_amd.workloads.transformer`` traces -- test infrastructure.

The same math as the traced graph: per-head projections on all rows,
per-sample attention scaled by 1/sqrt(d_model) with a softmax without max
subtraction, concat of samples then heads, output projection, post-norm
LayerNorm with biased variance and sqrt(|var + eps|), ReLU feed-forward,
MSE-to-zero loss (sum of out*out/numel), SGD ``p -= lr * grad``.

Run in-process on the CPU (``train``), or on the GPU in a child process
(``train_on_gpu``): a process that has loaded libadhip.so has the system
HIP runtime mapped, and torch's own HIP runtime then finds no device, so
the GPU run starts from a clean interpreter (``python -m
tests.torch_transformer in.npz out.npz``)."""
import os
import subprocess
import sys
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def flatten(res):
    """Parameters of a traced stack in a fixed order, with their ids:
    per layer wq[h], wk[h], wv[h] for each head, wo, the attention norm's
    scale and bias, the feed-forward's expand w, b and contract w, b, the
    feed-forward norm's scale and bias."""
    order = []
    for layer in res["net"]:
        att = layer.attention
        for i in range(att.num_heads):
            order += [att.wq[i].w, att.wk[i].w, att.wv[i].w]
        order.append(att.wo.w)
        order += [layer.layer_norm_att.scale, layer.layer_norm_att.bias]
        ff = layer.ffwd
        order += [ff.f_expand.w, ff.f_expand.b, ff.f_contract.w, ff.f_contract.b]
        order += [layer.layer_norm_ffwd.scale, layer.layer_norm_ffwd.bias]
    att = res["net"][0].attention
    shape = dict(layers=len(res["net"]), heads=att.num_heads, batch=att.batch, seq=att.seq,
                 d_model=att.d_model)
    return order, shape


def train(arrays, x, shape, steps, lr=0.01, device="cpu"):
    """``steps`` SGD steps from the parameters ``arrays`` (in ``flatten``
    order); returns them after the last step."""
    import torch
    torch.set_num_threads(max(1, min(16, torch.get_num_threads())))
    torch.backends.cuda.matmul.allow_tf32 = False
    p = [torch.tensor(a, device=device, requires_grad=True) for a in arrays]
    xt = torch.tensor(x, device=device)
    H, B, S, D = shape["heads"], shape["batch"], shape["seq"], shape["d_model"]
    per_layer = 3 * H + 1 + 2 + 4 + 2
    scale = 1.0 / np.sqrt(float(D))

    def ln(h, g, b):
        mean = h.mean(-1, keepdim=True)
        var = ((h - mean) ** 2).mean(-1, keepdim=True)
        return (h - mean) / torch.sqrt(torch.abs(var + 1e-5)) * g + b

    for _ in range(steps):
        out = xt
        for li in range(shape["layers"]):
            w = p[li * per_layer:(li + 1) * per_layer]
            heads = []
            for i in range(H):
                q, k, v = out @ w[3 * i], out @ w[3 * i + 1], out @ w[3 * i + 2]
                per = []
                for b in range(B):
                    rows = slice(b * S, (b + 1) * S)
                    e = torch.exp((q[rows] @ k[rows].T.contiguous()) * scale)
                    per.append((e / e.sum(-1, keepdim=True)) @ v[rows])
                heads.append(torch.cat(per, 0))
            o = 3 * H
            y = torch.cat(heads, -1) @ w[o]
            y = ln(out + y, w[o + 1], w[o + 2])
            h = torch.relu(y @ w[o + 3] + w[o + 4])
            z = h @ w[o + 5] + w[o + 6]
            out = ln(y + z, w[o + 7], w[o + 8])
        loss = (out * out * (1.0 / out.numel())).sum()
        for t in p:
            t.grad = None
        loss.backward()
        with torch.no_grad():
            for t in p:
                t -= lr * t.grad
    return [t.detach().cpu().numpy() for t in p]


def train_on_gpu(arrays, x, shape, steps, lr=0.01, timeout=600):
    """``train`` on cuda:0 in a child interpreter."""
    with tempfile.TemporaryDirectory() as tmp:
        src, dst = os.path.join(tmp, "in.npz"), os.path.join(tmp, "out.npz")
        np.savez(src, x=x, steps=steps, lr=lr, **{f"p{i}": a for i, a in enumerate(arrays)},
                 **{f"shape_{k}": v for k, v in shape.items()})
        r = subprocess.run([sys.executable, "-m", "tests.torch_transformer", src, dst], cwd=ROOT,
                           capture_output=True, text=True, timeout=timeout)
        if r.returncode != 0:
            raise RuntimeError(f"torch reference run failed ({r.returncode}):\n{r.stdout[-2000:]}\n{r.stderr[-4000:]}")
        with np.load(dst) as d:
            return [d[f"p{i}"] for i in range(len(arrays))]


def _main(src, dst):
    import torch
    if not torch.cuda.is_available():
        raise SystemExit("torch finds no GPU")
    with np.load(src) as d:
        n = sum(1 for k in d.files if k.startswith("p"))
        arrays = [d[f"p{i}"] for i in range(n)]
        shape = {k[6:]: int(d[k]) for k in d.files if k.startswith("shape_")}
        out = train(arrays, d["x"], shape, int(d["steps"]), float(d["lr"]), device="cuda:0")
    np.savez(dst, **{f"p{i}": a for i, a in enumerate(out)})


if __name__ == "__main__":
    _main(sys.argv[1], sys.argv[2])
