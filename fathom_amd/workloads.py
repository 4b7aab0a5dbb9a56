"""Seeded synthetic inputs for the five benchmark configurations of this path.

No model or dataset is available offline, so keys follow the distribution the
configurations specify: per KV head, channel scales sigma_c = exp(N(0, 1)) with
a few outlier channels x10, K = sigma * N(0, 1), query heads q ~ N(0, 1), and
planted keys at random positions set to 0.8 * q_g + N(0, (0.05 sigma)^2)
(planted key j targets head j mod G).  The calibration variance is the unbiased
per-channel variance over tokens >= 16 (scripts/sketch.py:52, SINK * 4).
Config 4 rotates channel pairs (c, c + 64) by pos * base^(-2c/128) with the
rotate-half convention of scripts/common.py:44-47.

The generator runs on the requested device with a torch.Generator seeded per
call, so the same seed on the same device gives the same bytes.
"""
import math

import torch

# Per-layer code-bit budgets of the 36-layer decode step (config 5): a fixed,
# seeded draw from [40, 92] (numpy default_rng(5), integers(40, 93)).
C5_BUDGETS = [75, 82, 41, 82, 64, 67, 73, 55, 91, 42, 54, 60, 70, 61, 46, 42, 40, 42,
              47, 92, 50, 74, 79, 52, 54, 63, 53, 91, 49, 87, 82, 84, 46, 60, 73, 66]

CONFIGS = {
    1: dict(name="C1 cpu-ref: 1 KV head, T=16384, fp16 query", BH=1, G=1, n=16384, k=128, sink=4, local=64,
            budget=48.0, outliers=4, planted=8, kdtype=torch.float32, qdtype=torch.float16, rope=None),
    2: dict(name="C2 Qwen3-8B layer, index in HBM: 8 KV heads, G=4, T=131072", BH=8, G=4, n=131072, k=512,
            sink=4, local=32, budget=48.0, outliers=4, planted=32, kdtype=torch.bfloat16, qdtype=torch.float32,
            rope=None),
    3: dict(name="C3 Qwen3-8B layer at 1M: 8 KV heads, G=4, T=1048576", BH=8, G=4, n=1048576, k=512, sink=4,
            local=32, budget=48.0, outliers=4, planted=32, kdtype=torch.bfloat16, qdtype=torch.float32, rope=None),
    4: dict(name="C4 Qwen2.5-7B layer: batch 2 x 4 KV heads, G=7, T=131072, RoPE keys", BH=8, G=7, n=131072,
            k=2048, sink=4, local=32, budget=48.0, budgets=(40.0, 48.0, 80.0), outliers=8, planted=32,
            kdtype=torch.bfloat16, qdtype=torch.float32, rope=1.0e6),
    5: dict(name="C5 Qwen3-8B decode step: 36 layers, batch 4 x 8 KV heads, G=4, T=32768", BH=32, G=4, n=32768,
            k=512, sink=4, local=32, budget=48.0, layers=36, outliers=4, planted=32, kdtype=torch.bfloat16,
            qdtype=torch.float32, rope=None),
}


def rope_rotate(K, base, pos0=0):
    """Rotate channel pairs (c, c + D/2) of K [BH, n, D] by pos * base^(-2c/D)
    (rotate-half convention, scripts/common.py:44-47)."""
    BH, n, d = K.shape
    half = d // 2
    pos = torch.arange(pos0, pos0 + n, device=K.device, dtype=torch.float64)
    inv = base ** (-torch.arange(half, device=K.device, dtype=torch.float64) * 2.0 / d)
    ang = pos[:, None] * inv[None, :]
    cos = torch.cos(ang).float()
    sin = torch.sin(ang).float()
    x1, x2 = K[..., :half], K[..., half:]
    return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], -1)


def synth_layer(BH, n, G, D=128, outliers=4, planted=32, seed=0, device="cpu", kdtype=torch.float32,
                qdtype=torch.float32, rope=None):
    """Keys, queries and calibration variance of one layer.

    Returns dict(K [BH, n, D] kdtype, q [BH, G, D] float32 (rounded through
    qdtype), var [BH, D] float32, planted [BH, planted] int64 positions)."""
    gen = torch.Generator(device=device).manual_seed(seed)
    sigma = torch.exp(torch.randn(BH, D, generator=gen, device=device))
    for b in range(BH):
        oc = torch.randperm(D, generator=gen, device=device)[:outliers]
        sigma[b, oc] *= 10.0
    K = torch.randn(BH, n, D, generator=gen, device=device) * sigma[:, None, :]
    q = torch.randn(BH, G, D, generator=gen, device=device).to(qdtype).float()
    npl = min(planted, max(n - 4 - 64, 0))
    pos = torch.zeros(BH, npl, dtype=torch.int64, device=device)
    for b in range(BH):
        p = torch.randperm(n - 4 - 64, generator=gen, device=device)[:npl] + 4
        pos[b] = p
        tgt = torch.arange(npl, device=device) % G
        noise = torch.randn(npl, D, generator=gen, device=device) * (0.05 * sigma[b])
        K[b, p] = 0.8 * q[b, tgt] + noise
    if rope:
        K = rope_rotate(K, rope)
    K = K.to(kdtype)
    var = K[:, 16:].float().var(1) if n > 17 else K.float().var(1)
    return {"K": K, "q": q, "var": var, "planted": pos}


def config_inputs(cfg_id, device="cpu", seed=0, n=None, BH=None, layer=0):
    """Inputs of configuration cfg_id (1-5), optionally with a smaller n or BH for
    parity tests.  For config 5, `layer` selects the layer (seed offset)."""
    c = dict(CONFIGS[cfg_id])
    if n is not None:
        c["n"] = n
    if BH is not None:
        c["BH"] = BH
    s = seed + (1000 * layer if cfg_id == 5 else 0)
    x = synth_layer(c["BH"], c["n"], c["G"], outliers=c["outliers"], planted=c["planted"], seed=s, device=device,
                    kdtype=c["kdtype"], qdtype=c["qdtype"], rope=c["rope"])
    if cfg_id == 5:
        c["budget"] = float(C5_BUDGETS[layer])
    c.update(x)
    c["g"] = ((c["q"] ** 2) * c["var"][:, None, :]).sum(1)
    return c


def synth_values(BH, n, D=128, seed=1, device="cpu", dtype=torch.bfloat16):
    gen = torch.Generator(device=device).manual_seed(seed)
    return torch.randn(BH, n, D, generator=gen, device=device).to(dtype)

