"""The sampler parity rule shared by the GPU tests: ids identical given the
same draws, except at a decision the oracle reports as within the precision
both sides carry.

  * greedy: the top-2 gap below 1e-5;
  * the p gap at the k-th place, or |r - cumsum| at the draw, below 1e-6:
    the GPU's exp/log (ocml, <= 1 ulp from glibc) move each p by ~1e-7
    relative, and the draw's sum2 / cumsum replay the reference's sequential
    order on those p;
  * the top-p cut (|cum - top_p| relative to top_p, or the relative p gap
    between the crossing id and the next) below 2e-5, or a p tie there: the
    reference normalises with a sequential f32 sum over the whole vocabulary
    (sampling.rs:154-167), whose own rounding error is ~1e-5 relative at
    50,257 ids (round-off of ~sqrt(n) adds, each up to half an ulp of a
    partial sum near the total); it scales every p by one common factor,
    which moves cum against top_p by that much.  The GPU's tree sum is closer
    to the exact normaliser, so a cut within that distance can fall on either
    side, and near-flat rows (GPT-2 bridge, thousands of ids at nearly equal
    p) put their cut between nearly tied ids.
"""

MARGIN_GREEDY = 1e-5
MARGIN_SAMPLED = 1e-6
MARGIN_TOP_P = 2e-5


def exempt(info, greedy):
    """True where the oracle's decision lies within the precision both sides carry."""
    if greedy:
        return info.greedy_gap < MARGIN_GREEDY
    return (info.topk_gap < MARGIN_SAMPLED or info.draw_gap < MARGIN_SAMPLED or info.topp_gap < MARGIN_TOP_P
            or bool(info.topp_tie))
