"""Seeded input generators for the parity tests and the benchmark.  TEST INFRASTRUCTURE ONLY.

Everything is drawn from a CPU ``torch.Generator`` (so values do not depend on
the device) and then moved.  Q, K, V are drawn in BTHD shape in that order and
returned as BHSD views over BTHD storage, as the reference's ``make_inputs``
does (benchmark/precision_check.py:120-130); dO is drawn after them in BTHD
shape (precision_check.py:284).

Config names follow BASELINE.json ``configs``:
  C  CPU plumbing      B1 Hq4 Hk2 T256 D64 fp32, causal
  H  headline          B1 T8192 Hq32 Hk8 D128 bf16
  P  packed documents  B2 T4096 Hq32 Hk8 D128 bf16, mask [B,1,T,T]
  S  score + mask      B1 T4096 Hq=Hk=16 D128 bf16, score/mask [B,Hq,T,T]
  M  MQA long KV       B1 Tq2048 Tk16384 Hq32 Hk1 D64 bf16, layout bshd
"""

from __future__ import annotations

from dataclasses import dataclass, field, replace
from typing import Optional

import torch


@dataclass(frozen=True)
class AttnConfig:
    name: str
    B: int
    Tq: int
    Tk: int
    Hq: int
    Hk: int
    D: int
    dtype: torch.dtype = torch.bfloat16
    is_causal: bool = False
    layout: str = "bhsd"
    mask: Optional[str] = None      # None | "bernoulli" | "packed_docs" | "sparse_diag"
    mask_heads: int = 0             # head extent of the generated mask (1 = broadcast)
    score: Optional[str] = None     # None | "normal" | "alibi_noise"
    keep_prob: float = 0.75
    score_scale: float = 0.1
    extra: dict = field(default_factory=dict, compare=False, hash=False)

    def scaled(self, **kw) -> "AttnConfig":
        return replace(self, **kw)


CONFIGS = {
    "C": AttnConfig("C", 1, 256, 256, 4, 2, 64, torch.float32, is_causal=True),
    "H": AttnConfig("H", 1, 8192, 8192, 32, 8, 128, torch.bfloat16),
    "H_causal": AttnConfig("H_causal", 1, 8192, 8192, 32, 8, 128, torch.bfloat16, is_causal=True),
    "P": AttnConfig("P", 2, 4096, 4096, 32, 8, 128, torch.bfloat16, mask="packed_docs", mask_heads=1),
    "S": AttnConfig("S", 1, 4096, 4096, 16, 16, 128, torch.bfloat16, mask="sparse_diag", mask_heads=16, score="alibi_noise"),
    "M": AttnConfig("M", 1, 2048, 16384, 32, 1, 64, torch.bfloat16, layout="bshd"),
}


def make_generator(seed: int) -> torch.Generator:
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    return g


def randn(shape, gen: torch.Generator, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    return torch.randn(shape, generator=gen, dtype=torch.float32).to(dtype)


def bernoulli_mask(B: int, H: int, Tq: int, Tk: int, keep_prob: float, gen: torch.Generator) -> torch.Tensor:
    """Bernoulli keep-mask with the diagonal (i, min(i, Tk-1)) forced to keep
    (precision_check.py:110-117)."""
    m = torch.rand((B, H, Tq, Tk), generator=gen) < keep_prob
    qi = torch.arange(Tq)
    m[:, :, qi, torch.clamp(qi, max=Tk - 1)] = True
    return m.contiguous()


def packed_docs_mask(B: int, T: int, gen: torch.Generator, lo: int = 128, hi: int = 1024) -> torch.Tensor:
    """[B, 1, T, T] block-diagonal causal mask of packed documents.

    Each sequence is cut into segments whose lengths are drawn uniformly from
    [lo, hi] (the last one truncated at T); keep iff same segment and j <= i.
    Every row keeps at least its diagonal.
    """
    seg = torch.empty((B, T), dtype=torch.long)
    for b in range(B):
        pos, sid = 0, 0
        while pos < T:
            n = int(torch.randint(lo, hi + 1, (1,), generator=gen).item())
            seg[b, pos:pos + n] = sid
            pos += n
            sid += 1
    same = seg[:, :, None] == seg[:, None, :]
    causal = torch.ones((T, T), dtype=torch.bool).tril()
    return (same & causal).unsqueeze(1).contiguous()


def sparse_diag_mask(B: int, H: int, Tq: int, Tk: int, drop_p: float, gen: torch.Generator) -> torch.Tensor:
    """Keys dropped i.i.d. with probability drop_p, diagonal always kept."""
    m = torch.rand((B, H, Tq, Tk), generator=gen) >= drop_p
    qi = torch.arange(Tq)
    m[:, :, qi, torch.clamp(qi, max=Tk - 1)] = True
    return m.contiguous()


def alibi_noise_score(B: int, H: int, Tq: int, Tk: int, gen: torch.Generator, noise_std: float = 0.1) -> torch.Tensor:
    """score[b,h,i,j] = -slope_h*|i-j| + N(0, noise_std), slope_h = 2^(-8(h+1)/H)."""
    slopes = torch.tensor([2.0 ** (-8.0 * (h + 1) / H) for h in range(H)], dtype=torch.float32)
    dist = (torch.arange(Tq)[:, None] - torch.arange(Tk)[None, :]).abs().float()
    s = -slopes.view(1, H, 1, 1) * dist.view(1, 1, Tq, Tk)
    s = s.expand(B, H, Tq, Tk) + torch.randn((B, H, Tq, Tk), generator=gen) * noise_std
    return s.contiguous()


def make_case(cfg: AttnConfig, seed: int = 0, device="cpu", with_grad: bool = True):
    """Inputs for one config: dict with q, k, v (in cfg.layout), mask, score,
    grad (same layout as q) and the BHSD views of all of them.

    The BHSD views (``*_bhsd``) are what the oracle consumes; ``q``/``k``/``v``/
    ``grad`` are what the product API receives for ``cfg.layout``.
    """
    gen = make_generator(seed)
    q = randn((cfg.B, cfg.Tq, cfg.Hq, cfg.D), gen, cfg.dtype)
    k = randn((cfg.B, cfg.Tk, cfg.Hk, cfg.D), gen, cfg.dtype)
    v = randn((cfg.B, cfg.Tk, cfg.Hk, cfg.D), gen, cfg.dtype)
    mask = None
    mh = cfg.mask_heads or cfg.Hq
    if cfg.mask == "bernoulli":
        mask = bernoulli_mask(cfg.B, mh, cfg.Tq, cfg.Tk, cfg.keep_prob, gen)
    elif cfg.mask == "packed_docs":
        assert cfg.Tq == cfg.Tk
        mask = packed_docs_mask(cfg.B, cfg.Tq, gen, **cfg.extra.get("packed", {}))
    elif cfg.mask == "sparse_diag":
        mask = sparse_diag_mask(cfg.B, mh, cfg.Tq, cfg.Tk, 0.1, gen)
    elif cfg.mask is not None:
        raise ValueError(cfg.mask)
    score = None
    if cfg.score == "normal":
        score = randn((cfg.B, cfg.Hq, cfg.Tq, cfg.Tk), gen) * cfg.score_scale
    elif cfg.score == "alibi_noise":
        score = alibi_noise_score(cfg.B, cfg.Hq, cfg.Tq, cfg.Tk, gen)
    elif cfg.score is not None:
        raise ValueError(cfg.score)
    grad = randn((cfg.B, cfg.Tq, cfg.Hq, cfg.D), gen, cfg.dtype) if with_grad else None

    def mv(x):
        return None if x is None else x.to(device)

    q, k, v, mask, score, grad = map(mv, (q, k, v, mask, score, grad))
    case = {
        "q_bhsd": q.transpose(1, 2),
        "k_bhsd": k.transpose(1, 2),
        "v_bhsd": v.transpose(1, 2),
        "grad_bhsd": None if grad is None else grad.transpose(1, 2),
        "mask": mask,
        "score": score,
    }
    if cfg.layout == "bhsd":
        case.update(q=case["q_bhsd"], k=case["k_bhsd"], v=case["v_bhsd"], grad=case["grad_bhsd"])
    else:
        case.update(q=q, k=k, v=v, grad=grad)
    return case
