"""Seeded synthetic workloads of the five benchmark configurations (C1-C5).

Each generator builds its tensors with a seeded torch.Generator on the target
device, so a run and its parity check see identical bits; ``scale`` shrinks the
token count for quick checks. ``algorithmic_bytes`` gives the compulsory HBM
traffic of one forward+backward pass that roofline fractions are computed from.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional

import torch
from torch import Tensor

IGNORE_INDEX = -100

C1 = dict(name="C1_rmsnorm", B=8, S=2048, H=4096, eps=1e-6, seed=0)
C2 = dict(name="C2_rope", B=8, S=2048, Hq=32, Hk=8, D=128, theta=500000.0, seed=1)
C3 = dict(name="C3_cross_entropy", N=16384, V=128256, ignore_frac=0.10, seed=2)
C4 = dict(name="C4_packed_varlen", T=32768, H=8192, Hq=64, Hk=8, D=128, theta=500000.0,
          min_doc=64, max_doc=4096, seed=3)
C5 = dict(name="C5_linear_ce", N=8192, H=4096, V=128256, ignore_frac=0.05, seed=4)


def _gen(device, seed: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _randn(shape, g, device, dtype=torch.bfloat16, std=1.0, mean=0.0) -> Tensor:
    t = torch.randn(shape, generator=g, device=device, dtype=torch.float32)
    if std != 1.0:
        t.mul_(std)
    if mean != 0.0:
        t.add_(mean)
    return t.to(dtype)


def _labels(n: int, v: int, ignore_frac: float, g, device) -> Tensor:
    labels = torch.randint(0, v, (n,), generator=g, device=device, dtype=torch.int64)
    n_ign = int(round(ignore_frac * n))
    if n_ign:
        idx = torch.randperm(n, generator=g, device=device)[:n_ign]
        labels[idx] = IGNORE_INDEX
    return labels


@dataclass
class Workload:
    name: str
    tensors: Dict[str, Tensor]
    params: Dict[str, object] = field(default_factory=dict)
    tokens: int = 0


def rmsnorm_workload(device, scale: float = 1.0, dtype=torch.bfloat16, H: Optional[int] = None,
                     cfg=C1, seed_offset: int = 0) -> Workload:
    B, S = cfg["B"], max(1, int(cfg["S"] * scale))
    H = H or cfg["H"]
    g = _gen(device, cfg["seed"] + seed_offset)
    x = _randn((B, S, H), g, device, dtype)
    w = _randn((H,), g, device, dtype, std=0.02, mean=1.0)
    dy = _randn((B, S, H), g, device, dtype)
    return Workload(cfg["name"], dict(x=x, w=w, dy=dy), dict(eps=cfg["eps"]), tokens=B * S)


def rope_workload(device, scale: float = 1.0, dtype=torch.bfloat16, cfg=C2,
                  seed_offset: int = 0) -> Workload:
    B, S = cfg["B"], max(1, int(cfg["S"] * scale))
    g = _gen(device, cfg["seed"] + seed_offset)
    q = _randn((B, S, cfg["Hq"], cfg["D"]), g, device, dtype)
    k = _randn((B, S, cfg["Hk"], cfg["D"]), g, device, dtype)
    dq = _randn((B, S, cfg["Hq"], cfg["D"]), g, device, dtype)
    dk = _randn((B, S, cfg["Hk"], cfg["D"]), g, device, dtype)
    return Workload(cfg["name"], dict(q=q, k=k, dq=dq, dk=dk),
                    dict(theta=cfg["theta"], S=S, D=cfg["D"]), tokens=B * S)


def ce_workload(device, scale: float = 1.0, dtype=torch.bfloat16, V: Optional[int] = None,
                cfg=C3, seed_offset: int = 0) -> Workload:
    N = max(1, int(cfg["N"] * scale))
    V = V or cfg["V"]
    g = _gen(device, cfg["seed"] + seed_offset)
    logits = _randn((N, V), g, device, dtype, std=2.0)
    labels = _labels(N, V, cfg["ignore_frac"], g, device)
    return Workload(cfg["name"], dict(logits=logits, labels=labels), dict(V=V), tokens=N)


def packed_doc_lengths(total: int, lo: int, hi: int, seed: int) -> List[int]:
    """Document lengths ~U{lo..hi} until they cover `total` tokens; the last one is truncated."""
    g = torch.Generator().manual_seed(seed)
    lens: List[int] = []
    covered = 0
    while covered < total:
        n = int(torch.randint(lo, hi + 1, (1,), generator=g))
        n = min(n, total - covered)
        lens.append(n)
        covered += n
    return lens


def packed_position_ids(lens: List[int]) -> Tensor:
    """position_ids that restart at 0 for every document (as pack_sequences emits them,
    packing.py:159-177 of the reference), int64 [1, sum(lens)]."""
    return torch.cat([torch.arange(n, dtype=torch.int64) for n in lens])[None, :]


def packed_workload(device, scale: float = 1.0, dtype=torch.bfloat16, cfg=C4) -> Workload:
    T = max(1, int(cfg["T"] * scale))
    lens = packed_doc_lengths(T, cfg["min_doc"], cfg["max_doc"], cfg["seed"])
    pos = packed_position_ids(lens).to(device)
    g = _gen(device, cfg["seed"])
    x = _randn((T, cfg["H"]), g, device, dtype)
    w = _randn((cfg["H"],), g, device, dtype, std=0.02, mean=1.0)
    dy = _randn((T, cfg["H"]), g, device, dtype)
    q = _randn((1, T, cfg["Hq"], cfg["D"]), g, device, dtype)
    k = _randn((1, T, cfg["Hk"], cfg["D"]), g, device, dtype)
    dq = _randn((1, T, cfg["Hq"], cfg["D"]), g, device, dtype)
    dk = _randn((1, T, cfg["Hk"], cfg["D"]), g, device, dtype)
    return Workload(cfg["name"], dict(x=x, w=w, dy=dy, q=q, k=k, dq=dq, dk=dk, position_ids=pos),
                    dict(theta=cfg["theta"], lens=lens, eps=1e-6, D=cfg["D"]), tokens=T)


def linear_ce_workload(device, scale: float = 1.0, dtype=torch.bfloat16, cfg=C5) -> Workload:
    N = max(1, int(cfg["N"] * scale))
    g = _gen(device, cfg["seed"])
    hidden = _randn((N, cfg["H"]), g, device, dtype)
    weight = _randn((cfg["V"], cfg["H"]), g, device, dtype, std=0.02)
    labels = _labels(N, cfg["V"], cfg["ignore_frac"], g, device)
    return Workload(cfg["name"], dict(hidden=hidden, weight=weight, labels=labels), {}, tokens=N)


# ---------------------------------------------------------------------------
# Compulsory HBM traffic of one forward+backward pass
# ---------------------------------------------------------------------------

def rmsnorm_bytes(rows: int, cols: int, elt: int = 2, w_elt: int = 2) -> Dict[str, int]:
    """fwd: read x, w; write y, rstd. bwd: read dy, x, w, rstd; write dx, dw."""
    x = rows * cols * elt
    fwd = 2 * x + cols * w_elt + rows * 4
    bwd = 3 * x + 2 * cols * w_elt + rows * 4
    return dict(fwd=fwd, bwd=bwd)


def add_rmsnorm_bytes(rows: int, cols: int, elt: int = 2, w_elt: int = 2) -> int:
    """Fused residual add + RMSNorm forward: read x, residual, w; write y, h, rstd."""
    return 4 * rows * cols * elt + cols * w_elt + rows * 4


def swiglu_bytes(n: int, elt: int = 2) -> Dict[str, int]:
    """fwd: read gate, up; write out. bwd: read dout, gate, up; write dgate, dup."""
    return dict(fwd=3 * n * elt, bwd=5 * n * elt)


def rope_bytes(tokens: int, heads: int, D: int, elt: int = 2, pos_bytes: int = 0) -> Dict[str, int]:
    """fwd and bwd each read and write every Q/K element once (+ position_ids)."""
    t = tokens * heads * D * elt
    return dict(fwd=2 * t + pos_bytes, bwd=2 * t + pos_bytes)


def ce_bytes(n: int, n_valid: int, v: int, elt: int = 2) -> Dict[str, int]:
    """fwd reads the rows with a label (ignored rows are not read); bwd reads those
    rows and writes every row's gradient. Labels (8 B/row), loss and lse (4 B/row each)."""
    row = v * elt
    fwd = n_valid * row + n * (8 + 4 + 4)
    bwd = n_valid * row + n * row + n * (8 + 4 + 4)
    return dict(fwd=fwd, bwd=bwd)


def ce_bytes_fused(n: int, n_valid: int, v: int, elt: int = 2) -> int:
    """Schedule B (loss and gradient in one pass): read every row with a label once,
    write every row's gradient once; labels, loss and lse per row."""
    return n_valid * v * elt + n * v * elt + n * (8 + 4 + 4)


def vocab_shard_bytes(n: int, vp: int, p: int, elt: int = 2) -> Dict[str, int]:
    """One rank of a P-way vocabulary-parallel CE over a [n, vp] shard. stats: read
    the shard and the targets, write 16 B of partials per row. merge: read the P
    ranks' partials, write lse and loss. bwd: read the shard, targets and lse, write
    the gradient."""
    shard = n * vp * elt
    return dict(stats=shard + n * (8 + 16), merge=p * n * 16 + n * 8,
                bwd=2 * shard + n * (8 + 4) + 4)


def linear_ce_flops(n: int, h: int, v: int) -> int:
    """Three GEMMs of 2*N*V*H: logits, grad_hidden, grad_weight."""
    return 3 * 2 * n * v * h
