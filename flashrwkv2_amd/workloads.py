"""Seeded synthetic inputs for the benchmark configurations of the WKV7 path.

Distributions (per element unless noted):
  r, k, v ~ N(0, 1)
  decay: u ~ U(lo, hi) with hi <= -1/2, and the reference's logit contract
         decay_logits = logit(exp(u + 1/2)), evaluated in fp64 and rounded to
         the token dtype.  Then exp(-exp(-1/2) * sigmoid(decay_logits)) =
         exp(-exp(u)) = w, the requested retention.
  kk = L2-normalise(N(0, 1)) over D, per (token, head);  a = -kk;
  b  = kk * sigmoid(N(0, 1))
  initial state (when present) ~ N(0, 0.1^2) (standard deviation 0.1)

Everything is drawn in fp64 from one ``torch.Generator`` seeded per config
(on the target device, so the large configurations need no host staging) and
rounded to the token dtype once.  Consumers that need the exact kernel inputs
read them back from the returned tensors.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

HEAD_SIZE = 64


@dataclass
class Workload:
    name: str
    r: torch.Tensor
    decay_logits: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    a: torch.Tensor
    b: torch.Tensor
    cu_seqlens: torch.Tensor       # int32 [N+1]
    state_indices: torch.Tensor    # int32 [N]
    state_pool: torch.Tensor       # fp32 [N,H,D,D]
    max_seqlen: int
    info: dict = field(default_factory=dict)

    @property
    def tokens(self) -> tuple[torch.Tensor, ...]:
        return (self.r, self.decay_logits, self.k, self.v, self.a, self.b)

    @property
    def total_tokens(self) -> int:
        return int(self.r.shape[0])

    @property
    def num_heads(self) -> int:
        return int(self.r.shape[1])


def decay_logits_for(u: torch.Tensor) -> torch.Tensor:
    """logit(exp(u + 1/2)) in fp64; requires u < -1/2."""
    p = torch.exp(u.double() + 0.5).clamp_(max=1.0 - 2.0**-40)
    return torch.log(p) - torch.log1p(-p)


def make_tokens(total: int, heads: int, *, u_range: tuple[float, float], seed: int,
                device: torch.device | str, dtype: torch.dtype = torch.bfloat16,
                head_size: int = HEAD_SIZE):
    """r, decay_logits, k, v, a, b of shape [total, heads, head_size]."""
    dev = torch.device(device)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    shape = (total, heads, head_size)

    def normal():
        return torch.randn(shape, generator=g, device=dev, dtype=torch.float64)

    r = normal().to(dtype)
    k = normal().to(dtype)
    v = normal().to(dtype)
    lo, hi = u_range
    if not hi <= -0.5:
        raise ValueError("u must stay below -1/2 for the logit contract")
    u = torch.rand(shape, generator=g, device=dev, dtype=torch.float64) * (hi - lo) + lo
    decay_logits = decay_logits_for(u).to(dtype)
    del u
    kk = normal()
    kk = kk / kk.norm(dim=-1, keepdim=True)
    gate = torch.sigmoid(normal())
    a = (-kk).to(dtype)
    b = (kk * gate).to(dtype)
    return r, decay_logits, k, v, a, b


def _state(n: int, heads: int, seed: int, device, std: float | None):
    dev = torch.device(device)
    if std is None:
        return torch.zeros((n, heads, HEAD_SIZE, HEAD_SIZE), device=dev, dtype=torch.float32)
    g = torch.Generator(device=dev)
    g.manual_seed(seed + 7919)
    return (torch.randn((n, heads, HEAD_SIZE, HEAD_SIZE), generator=g, device=dev,
                        dtype=torch.float32) * std)


def _pack(name, toks, lengths, heads, state_std, seed, device, info):
    dev = torch.device(device)
    offsets = [0]
    for n in lengths:
        offsets.append(offsets[-1] + int(n))
    cu = torch.tensor(offsets, device=dev, dtype=torch.int32)
    n = len(lengths)
    idx = torch.arange(n, device=dev, dtype=torch.int32)
    pool = _state(n, heads, seed, dev, state_std)
    return Workload(name, *toks, cu, idx, pool, max(int(x) for x in lengths), info)


def config(idx: int, device="cuda", *, dtype=torch.bfloat16, batch=None, tokens=None,
           heads=None, sequences=None, max_len=None) -> Workload:
    """BASELINE config ``idx`` (0..4); keyword overrides shrink it for tests."""
    if idx == 0:
        B, T, H = batch or 1, tokens or 64, heads or 4
        toks = make_tokens(B * T, H, u_range=(-6.0, -0.5), seed=1000, device=device,
                           dtype=dtype)
        return _pack("cfg0_cpu_ref_B1_T64_H4", toks, [T] * B, H, None, 1000, device,
                     {"B": B, "T": T, "H": H})
    if idx == 1:
        B, T, H = batch or 8, tokens or 4096, heads or 32
        toks = make_tokens(B * T, H, u_range=(-6.0, -0.5), seed=1001, device=device,
                           dtype=dtype)
        return _pack(f"cfg1_prefill_B{B}_T{T}_H{H}", toks, [T] * B, H, None, 1001, device,
                     {"B": B, "T": T, "H": H})
    if idx == 2:
        N, H = batch or 256, heads or 32
        toks = make_tokens(N, H, u_range=(-6.0, -0.5), seed=1002, device=device, dtype=dtype)
        return _pack(f"cfg2_decode_N{N}_H{H}", toks, [1] * N, H, 0.1, 1002, device,
                     {"N": N, "T": 1, "H": H})
    if idx == 3:
        S, H, L = sequences or 64, heads or 64, max_len or 2048
        g = torch.Generator()
        g.manual_seed(1003)
        lengths = torch.randint(1, L + 1, (S,), generator=g).tolist()
        toks = make_tokens(sum(lengths), H, u_range=(-6.0, -0.5), seed=1003, device=device,
                           dtype=dtype)
        return _pack(f"cfg3_varlen_S{S}_H{H}", toks, lengths, H, 0.1, 1003, device,
                     {"S": S, "H": H, "sum_T": sum(lengths)})
    if idx == 4:
        T, H = tokens or 65536, heads or 64
        toks = make_tokens(T, H, u_range=(-9.0, -4.0), seed=1004, device=device, dtype=dtype)
        return _pack(f"cfg4_long_T{T}_H{H}", toks, [T], H, None, 1004, device,
                     {"B": 1, "T": T, "H": H})
    raise ValueError(f"unknown config {idx}")
