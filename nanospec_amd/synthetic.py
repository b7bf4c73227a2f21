"""Seeded synthetic inputs for the benchmark configurations C0-C4.

Distributions follow the benchmark definitions (draw order: hidden -> W_lm ->
Markov -> draft logits -> teacher logits -> peaks -> agreement -> labels ->
masks; seed 1000 + config index; fp32 draws cast to bf16).  Inputs are made
on the target device with torch's generator: this is input plumbing, not part
of the measured path.

``Slots`` duck-types the reference's PreparedBatch for the objective: it has
``weights`` (fp32), ``target_ids`` (int64) and ``valid`` (bool), each
[blocks, K] (dspark.py:95-106, 116-127).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

VOCAB = 248_320        # DraftConfig.vocab_size (config.py:17)
HIDDEN = 5_120         # DraftConfig.hidden_size (config.py:11)
BLOCK = 8              # slots per anchor block in every configuration


@dataclass
class Slots:
    weights: torch.Tensor
    target_ids: torch.Tensor
    valid: torch.Tensor


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def rms_normalise(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)


def position_weights(valid: torch.Tensor, gamma: float) -> torch.Tensor:
    """valid * exp(-slot / gamma), no decay when gamma <= 0 (dspark.py:124-126)."""
    w = valid.float()
    if gamma > 0:
        slot = torch.arange(valid.shape[-1], device=valid.device, dtype=torch.float32)
        w = w * torch.exp(-slot / gamma)
    return w


def _peaked(n, v, scale, peak, g, device, at=None):
    x = scale * torch.randn((n, v), generator=g, device=device, dtype=torch.float32)
    if at is None:
        at = torch.randint(0, v, (n,), generator=g, device=device)
    x[torch.arange(n, device=device), at] += peak
    return x, at


def _teacher(n, v, g, device):
    """3 N(0,1) + 8 at one uniformly random token per row."""
    return _peaked(n, v, 3.0, 8.0, g, device)[0].to(torch.bfloat16)


def _labels(n, v, g, device):
    return torch.randint(0, v, (n,), generator=g, device=device)


def head_inputs(n, d, v, seed, device, *, ragged=False, gamma=4.0, k=BLOCK):
    """Fused-path inputs (C0, C2, C3 recipe): hidden, W_lm, Markov logits, teacher, Slots."""
    g = _gen(seed, device)
    hidden = rms_normalise(torch.randn((n, d), generator=g, device=device)).to(torch.bfloat16)
    weight = (0.02 * torch.randn((v, d), generator=g, device=device)).to(torch.bfloat16)
    markov = (0.5 * torch.randn((n, v), generator=g, device=device)).to(torch.bfloat16)
    teacher = _teacher(n, v, g, device)
    labels = _labels(n, v, g, device)
    nb = n // k
    if ragged:
        lengths = torch.randint(1, k + 1, (nb, 1), generator=g, device=device)
        valid = torch.arange(k, device=device).unsqueeze(0) < lengths
    else:
        valid = torch.ones((nb, k), dtype=torch.bool, device=device)
    slots = Slots(position_weights(valid, gamma), labels.view(nb, k), valid)
    return hidden, weight, markov, teacher, slots


def markov_factors(n, v, r, seed, device):
    """Factored Markov head (MarkovHead, layers.py:74-78): previous ids ~ U[0, V),
    w1 ~ N(0, 1), w2 ~ N(0, 0.05) (bf16), so w1[prev] . w2^T has std about
    0.05 sqrt(r) (0.8 at r = 256, like the dense recipe's N(0, 0.5))."""
    g = _gen(seed, device)
    prev = torch.randint(0, v, (n,), generator=g, device=device)
    w1 = torch.randn((v, r), generator=g, device=device).to(torch.bfloat16)
    w2 = (0.05 * torch.randn((v, r), generator=g, device=device)).to(torch.bfloat16)
    return prev, w1, w2


def c0(device="cpu"):
    """C0 CPU plumbing: N = 64 (8 x 8), d = 256, V = 8192, gamma 4, all valid."""
    return head_inputs(64, 256, 8192, 1000, device)


def logits_inputs(n, v, seed, device, *, k=BLOCK, gamma=4.0, masked_fraction=0.1, agree=0.6):
    """C1 recipe: draft 2 N(0,1) + 6 at peak_d, teacher 3 N(0,1) + 8 at peak_t,
    peak_t = peak_d on `agree` of rows, floor(masked_fraction N) rows masked."""
    g = _gen(seed, device)
    draft, peak_d = _peaked(n, v, 2.0, 6.0, g, device)
    draft = draft.to(torch.bfloat16)
    teacher = 3.0 * torch.randn((n, v), generator=g, device=device)
    other = torch.randint(0, v, (n,), generator=g, device=device)
    same = torch.rand((n,), generator=g, device=device) < agree
    peak_t = torch.where(same, peak_d, other)
    teacher[torch.arange(n, device=device), peak_t] += 8.0
    teacher = teacher.to(torch.bfloat16)
    labels = _labels(n, v, g, device)
    keep = torch.ones(n, dtype=torch.bool, device=device)
    masked = torch.randperm(n, generator=g, device=device)[: int(masked_fraction * n)]
    keep[masked] = False
    valid = keep.view(n // k, k)
    slots = Slots(position_weights(valid, gamma), labels.view(n // k, k), valid)
    return draft, teacher, slots


def c1(device, n=4096, v=VOCAB):
    return logits_inputs(n, v, 1001, device)


def c2(device, n=4096, d=HIDDEN, v=VOCAB):
    return head_inputs(n, d, v, 1002, device)


def c3(device, n=32768, d=HIDDEN, v=VOCAB):
    return head_inputs(n, d, v, 1003, device, ragged=True, gamma=2.0)


def fp8_teacher_inputs(n, d, v, seed, device):
    """C4 teacher head: hidden ~N(0,1) bf16 and W_t ~N(0, 0.02) quantised to
    e4m3 with one fp32 scale per 128x128 block (s = amax / 448)."""
    if v % 128 or d % 128:
        raise ValueError("FP8 teacher head needs V and d multiples of 128")
    g = _gen(seed, device)
    x = torch.randn((n, d), generator=g, device=device).to(torch.bfloat16)
    w = 0.02 * torch.randn((v, d), generator=g, device=device)
    blocks = w.view(v // 128, 128, d // 128, 128)
    scale = blocks.abs().amax(dim=(1, 3)) / 448.0
    q = (blocks / scale.clamp_min(torch.finfo(torch.float32).tiny)[:, None, :, None]).clamp(-448, 448)
    codes = q.to(torch.float8_e4m3fn).view(v, d).view(torch.uint8)
    return x, codes.contiguous(), scale.contiguous()


def c4(device, n=4096, d=HIDDEN, v=VOCAB):
    hidden, weight, markov, _, slots = head_inputs(n, d, v, 1004, device)
    x, codes, scale = fp8_teacher_inputs(n, d, v, 2004, device)
    return hidden, weight, markov, (x, codes, scale), slots
