"""Routing parity in bf16, proven token by token.

The reference computes the router logits with a bf16 Linear and a bf16
softmax on the CPU (aspa.py:149-157), then the prototype prior in f32
(aspa.py:628-690) and torch.topk over the head probabilities
(aspa.py:1590-1591).  The HIP router computes the same f32 dot products in
another order.  Two things can therefore make a token's head set differ
from the reference's:

1. a tie: the reference's k-th and (k+1)-th head probabilities are equal
   and torch.topk on the CPU keeps a higher index, where this build keeps
   the lowest (the tie rule of the north star);
2. a bf16 rounding boundary: an exact logit (or a softmax output) sits so
   close to the midpoint between two bf16 numbers that the two f32
   evaluation orders round it to different neighbours.

check_routing() asserts that every difference is one of these two: the
head sets equal topk_lowest(reference gate probabilities) on every token
whose gate probabilities equal the reference's bit for bit, and every token
whose gate probabilities differ sits at a bf16 rounding boundary.  On those
boundary tokens the head sets are compared too: a set can only differ there
when the rounding difference is large enough to reorder the reference's
k-th and (k+1)-th head probabilities, i.e. when their gap is at most twice
the token's largest gate difference (a near-tie); every differing boundary
set must satisfy that, and the number of them is counted and bounded by
the caller.  It returns the counts so that tests can report them.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch
import torch.nn.functional as F

from oracle import aspa_oracle as O

# A logit within 2^-9 bf16 ulps of a rounding boundary (2^7 f32 ulps: the
# spread of f32 dot products of 512 terms summed in different orders), or a
# softmax output within 2^-12 bf16 ulps (2^4 f32 ulps: exp/sum/divide
# rounding), counts as "at a boundary".
LOGIT_TOL = 2.0 ** -9
SOFTMAX_TOL = 2.0 ** -12


def bf16_boundary_distance(z: np.ndarray) -> np.ndarray:
    """Distance of each value to the nearest bf16 rounding boundary (the
    midpoint between two adjacent bf16 numbers), in bf16 ulps of its binade
    (0 = exactly on a midpoint, 0.5 = exactly on a bf16 number)."""
    a = np.abs(np.asarray(z, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(a, 1e-38)))
    ulp = np.exp2(e - 7.0)
    frac = np.mod(a / ulp, 1.0)
    return np.abs(frac - 0.5)


@dataclass
class RoutingReport:
    tokens: int
    ties: int            # head set differs from the reference's; its probs tie at the boundary
    gate_diff: int       # gate probabilities differ from the reference's (all at a boundary)
    base_rate: float     # fraction of all tokens that would pass the boundary test
    boundary_set_diff: int = 0  # boundary tokens whose head set differs (each a near-tie)

    def __str__(self) -> str:
        return (f"{self.tokens} tokens: {self.ties} tie(s) broken to the lowest head index, "
                f"{self.gate_diff} token(s) with gate probs at a bf16 rounding boundary, "
                f"{self.boundary_set_diff} of them with a different head set (near-ties) "
                f"(boundary base rate {self.base_rate:.4f})")

    def assert_boundary_sets_at_most(self, frac: float, floor: int = 2) -> None:
        """Bound the head-set differences on boundary tokens: at most
        max(floor, frac * tokens)."""
        bound = max(int(floor), int(frac * self.tokens))
        assert self.boundary_set_diff <= bound, (
            f"{self.boundary_set_diff} boundary tokens with a different head set (bound {bound})")


def _at_boundary(x_bf16: torch.Tensor, w_bf16: torch.Tensor) -> np.ndarray:
    """(n,) bool: some exact logit, or some softmax output of the bf16
    logits, of the token lies at a bf16 rounding boundary."""
    exact = (x_bf16.double() @ w_bf16.double().t()).numpy()
    logits = F.linear(x_bf16, w_bf16).double()
    p = torch.softmax(logits, dim=-1).numpy()
    return (bf16_boundary_distance(exact) <= LOGIT_TOL).any(-1) | (bf16_boundary_distance(p) <= SOFTMAX_TOL).any(-1)


def check_routing(ours_sets: torch.Tensor, ref_sets: torch.Tensor, ours_gate: torch.Tensor, ref_gate: torch.Tensor,
                  x_bf16: torch.Tensor, w_bf16: torch.Tensor, k: int,
                  token_mask: torch.Tensor = None, gate_to_head: torch.Tensor = None,
                  sum_ulps: int = 0) -> RoutingReport:
    """ours_sets / ref_sets: (n, H) bool head sets; ours_gate / ref_gate:
    (n, G) f32; gate_to_head (G,) the gate -> head map (None: G == H, the
    identity map), the head probabilities being the gates summed per head
    (aspa.py:675-690); x_bf16 (n, C), w_bf16 (G, C) the router's operands;
    token_mask (n,) bool or None (a masked token has an empty set on both
    sides).  sum_ulps: gates that differ by at most that many f32 ulps of 1
    are explained by the order of the f32 sum that renormalises the gates
    with the prototype prior on (aspa.py:667-670: G bf16 terms, exact with 8
    gates, not with 32 or 64); their head sets are judged like those of
    boundary tokens."""
    n = ours_sets.size(0)
    same_gate = (ours_gate == ref_gate).all(-1)
    in_sum = (ours_gate - ref_gate).abs().amax(-1) <= float(sum_ulps) * 2.0 ** -24
    if gate_to_head is not None:
        H = ours_sets.size(1)
        ours_gate = O.head_probs_from_gates(ours_gate, gate_to_head, H)
        ref_gate = O.head_probs_from_gates(ref_gate, gate_to_head, H)
    at_b = torch.from_numpy(_at_boundary(x_bf16, w_bf16))
    unexplained_gate = (~same_gate) & (~at_b) & (~in_sum)
    assert int(unexplained_gate.sum()) == 0, (
        f"gate probabilities differ away from a bf16 rounding boundary at tokens "
        f"{torch.nonzero(unexplained_gate).flatten()[:20].tolist()}")
    # where the gates agree bit for bit, the head set is exactly the lowest-index top-k of the reference's gates
    _, idx = O.topk_lowest(ref_gate, k)
    exp = torch.zeros_like(ours_sets)
    exp.scatter_(1, idx, True)
    if token_mask is not None:
        exp &= token_mask.view(-1, 1)
    wrong = same_gate & (ours_sets != exp).any(-1)
    assert int(wrong.sum()) == 0, f"head sets differ from topk_lowest(reference gates) at {torch.nonzero(wrong).flatten()[:20].tolist()}"
    # every token whose set differs from the reference's own choice is a tie
    # at the boundary of the reference's gates (or a boundary token)
    srt = torch.sort(ref_gate, dim=-1, descending=True).values
    tie = srt[:, k - 1] == srt[:, k]
    differs = (ours_sets != ref_sets).any(-1)
    if token_mask is not None:
        differs &= token_mask
    unexplained_set = differs & ~tie & same_gate
    assert int(unexplained_set.sum()) == 0, f"head sets differ without a tie at {torch.nonzero(unexplained_set).flatten()[:20].tolist()}"
    # boundary tokens: a different head set needs the rounding difference to
    # reorder the reference's k-th and (k+1)-th probabilities
    bdiff = differs & ~same_gate
    gap = (srt[:, k - 1] - srt[:, k]).double()
    dmax = (ours_gate.double() - ref_gate.double()).abs().amax(-1)
    far = bdiff & (gap > 2.0 * dmax)
    assert int(far.sum()) == 0, (
        f"head sets differ on boundary tokens whose k-th/(k+1)-th gap exceeds the rounding difference at "
        f"{torch.nonzero(far).flatten()[:20].tolist()}")
    return RoutingReport(tokens=n, ties=int((differs & same_gate).sum()), gate_diff=int((~same_gate).sum()),
                         base_rate=float(at_b.float().mean()), boundary_set_diff=int(bdiff.sum()))
