"""Seeded synthetic inputs of the BASELINE configurations, generated on the device (for
``bench.py`` and the tests; nothing of the encode path reads them).

* :func:`zipf_topk`: the cfg5 router (OLMoE-shaped layer: 64 experts, top-8 of 16384
  tokens with Zipf(1.1)-skewed expert load).  Each token picks ``topk`` distinct experts
  by Gumbel-top-k on log Zipf weights (sampling without replacement in proportion to
  the weights), so an expert sees at most one slot per token.
* :func:`activations`: bf16 calibration tokens, N(0, 1) with 1 % of the channels (a
  seeded choice) scaled x20 (the outlier recipe of every configuration).
"""

import torch


def zipf_topk(tokens: int, experts: int, topk: int, s: float = 1.1, seed: int = 0,
              device="cuda") -> torch.Tensor:
    """``[tokens, topk]`` int64 expert indices: expert popularity rank r (a seeded
    permutation of the experts) has weight (r + 1)^-s; each token draws ``topk``
    distinct experts by Gumbel-top-k."""
    g = torch.Generator(device=device).manual_seed(seed)
    rank = torch.randperm(experts, generator=g, device=device)
    logw = -s * torch.log((rank + 1).to(torch.float32))
    u = torch.rand(tokens, experts, generator=g, device=device).clamp_min(1e-30)
    keys = logw[None, :] - torch.log(-torch.log(u))
    return torch.topk(keys, topk, dim=-1).indices.to(torch.int64)


def activations(t: int, k: int, seed: int, device="cuda") -> torch.Tensor:
    """``[t, k]`` bf16: N(0, 1) with 1 % of the channels x20."""
    g = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn(t, k, generator=g, device=device)
    x[:, torch.randperm(k, generator=g, device=device)[: -(-k // 100)]] *= 20.0
    return x.to(torch.bfloat16)
