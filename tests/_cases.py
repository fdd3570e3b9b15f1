"""Seeded attention test cases and the tolerance checks shared by the CPU and GPU tests.

Tolerances (stated once, used everywhere):
* f64 inputs:  max |out - ref| <= 1e-10 and max |lse - ref| <= 1e-10 (the reference's own
  sequence-parallel tests use 1e-12 on f64 results of the same algorithm; kernels with a
  different summation order are held to 1e-10);
* f32 inputs:  normwise rel <= 1e-5 on out and on lse, i.e. max|a-b| / max|ref|;
* bf16 / f16 inputs (f32 accumulation): max |out - ref| <= 2e-2, max |lse - ref| <= 1e-3;
* rows without a visible key: out exactly 0 and lse exactly -inf, at the same rows as the
  reference (never NaN).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Sequence, Tuple

import torch


def make_positions(kind: str, B: int, Sq: int, Sk: int, g: torch.Generator):
    """(q_pos, k_pos) for one of the mask patterns the reference supports."""
    if kind == "aligned":          # causal prefill without padding (mode 'causal')
        assert Sq == Sk
        p = torch.arange(Sq).repeat(B, 1)
        return p, p.clone()
    if kind == "left_pad":         # tests/test_sequence_parallel.py:23-25
        assert Sq == Sk
        p = torch.arange(Sq).repeat(B, 1)
        pad = min(3, Sq - 1)
        p[-1, :pad] = -1
        p[-1, pad:] -= pad
        return p, p.clone()
    if kind == "right_pad":        # packed tokens then padding (engine.py:328-329)
        assert Sq == Sk
        p = torch.arange(Sq).repeat(B, 1)
        p[:, Sq - max(1, Sq // 5):] = -1
        return p, p.clone()
    if kind == "zigzag":           # queries of two far-apart chunks against a later block
        half = Sq // 2
        qp = torch.cat([torch.arange(half), torch.arange(3 * Sk, 3 * Sk + Sq - half)]).repeat(B, 1)
        kp = (torch.arange(Sk) + Sk).repeat(B, 1)
        return qp, kp
    if kind == "decode":           # one new token per sequence against a -1-tailed cache
        lens = torch.randint(1, Sk + 1, (B,), generator=g)
        slots = torch.arange(Sk).view(1, Sk)
        kp = torch.where(slots < lens.view(-1, 1), slots, torch.full_like(slots, -1))
        qp = (lens - 1).view(-1, 1) + torch.arange(Sq).view(1, Sq) * 0
        return qp, kp
    if kind == "random":           # arbitrary order, some padding
        qp = torch.randint(-1, 2 * Sk, (B, Sq), generator=g)
        kp = torch.randint(-1, 2 * Sk, (B, Sk), generator=g)
        return qp, kp
    if kind == "all_pad":          # every key invalid
        return torch.arange(Sq).repeat(B, 1), torch.full((B, Sk), -1)
    raise ValueError(kind)


@dataclass
class Case:
    B: int
    Sq: int
    Sk: int
    Hq: int
    Hkv: int
    D: int
    kind: str = "aligned"
    causal: bool = True
    kv_map: Optional[Tuple[int, ...]] = None
    scale: Optional[float] = None
    seed: int = 0

    def tensors(self, dtype: torch.dtype):
        g = torch.Generator().manual_seed(self.seed)
        q = torch.randn(self.B, self.Sq, self.Hq, self.D, generator=g).to(dtype)
        k = torch.randn(self.B, self.Sk, self.Hkv, self.D, generator=g).to(dtype)
        v = torch.randn(self.B, self.Sk, self.Hkv, self.D, generator=g).to(dtype)
        qp, kp = make_positions(self.kind, self.B, self.Sq, self.Sk, g)
        return q, k, v, qp, kp

    def __str__(self):
        return (f"B{self.B}-Sq{self.Sq}-Sk{self.Sk}-H{self.Hq}/{self.Hkv}-D{self.D}-{self.kind}"
                f"-{'c' if self.causal else 'nc'}" + (f"-map{self.kv_map}" if self.kv_map else "")
                + (f"-s{self.scale}" if self.scale is not None else ""))


def tolerances(dtype: torch.dtype):
    if dtype == torch.float64:
        return ("abs", 1e-10, 1e-10)
    if dtype == torch.float32:
        return ("rel", 1e-5, 1e-5)
    return ("abs", 2e-2, 1e-3)


def assert_attention_close(out, lse, ref_out, ref_lse, dtype, what=""):
    """Checks (out, lse) against the reference result with the tolerances above."""
    out, ref_out = out.detach().cpu().double(), ref_out.detach().cpu().double()
    assert out.shape == ref_out.shape, (what, out.shape, ref_out.shape)
    mode, tol_o, tol_l = tolerances(dtype)
    assert torch.isfinite(out).all(), f"{what}: non-finite output"
    if lse is not None:
        lse, ref_lse = lse.detach().cpu().double(), ref_lse.detach().cpu().double()
        fin = torch.isfinite(ref_lse)
        assert torch.equal(torch.isfinite(lse), fin), f"{what}: empty-row pattern differs"
        assert not torch.isnan(lse).any(), f"{what}: NaN lse"
        assert (lse[~fin] == float("-inf")).all(), f"{what}: empty rows must have lse = -inf"
        empty = (~fin).transpose(1, 2)  # [B, Sq, H]
        assert (out[empty] == 0).all(), f"{what}: empty rows must be exactly 0"
        if fin.any():
            dl = (lse[fin] - ref_lse[fin]).abs().max().item()
            if mode == "rel":
                dl /= max(ref_lse[fin].abs().max().item(), 1e-30)
            assert dl <= tol_l, f"{what}: lse error {dl:.3e} > {tol_l}"
    do = (out - ref_out).abs().max().item() if out.numel() else 0.0
    if mode == "rel":
        do /= max(ref_out.abs().max().item(), 1e-30) if out.numel() else 1.0
    assert do <= tol_o, f"{what}: out error {do:.3e} > {tol_o}"
    return do
