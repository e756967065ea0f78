"""Token-stream parity between two backends of the paged engine, with the evidence that
explains every divergence.

Greedy streams from ATTENTION=hip and ATTENTION=gather (the reference path) run the
same model, weights and requests. In half precision their logits differ by rounding
(the kernels accumulate in another order), so a stream may part from the reference
where the reference's own top logits are (near-)tied. `MarginProbe` makes that
checkable: it is installed as the gather engine's `PagedExecutor.logit_probe` and,
at every step, measures how far below the step's maximum logit the candidate
stream's token sits, in units in the last place of the logit dtype. Up to a stream's
first divergence both runs fed the same history, so at the divergence the distance is
exactly "how close to a tie the reference was". A divergence at a clear margin is a
bug, not rounding.

The reference samples `logits[0, ends - 1, :].argmax(-1)`
(inference_server/core/paged_executor.py:194-203), which is the distance-0 token.
"""

from __future__ import annotations

import torch

_MAG = {torch.float16: (torch.int16, 0x7FFF), torch.bfloat16: (torch.int16, 0x7FFF),
        torch.float32: (torch.int32, 0x7FFFFFFF)}


def ordinal(x: torch.Tensor) -> torch.Tensor:
    """Order-preserving integer image of floats (int64): consecutive representable
    values of x's dtype map to consecutive integers and +0 / -0 both map to 0, so the
    difference of two images is a distance in ulps."""
    ity, mag = _MAG[x.dtype]
    u = x.view(ity).to(torch.int64)
    return torch.where(u < 0, -(u & mag), u)


class MarginProbe:
    """`logit_probe` for an engine run: records, for each (sequence id, token index)
    at which a candidate stream has a token, the ulp distance between the step's
    maximum logit and the candidate token's logit. One probe serves several
    candidate streams (name -> {seq_id: tokens})."""

    def __init__(self, candidates: dict[str, dict[str, list[int]]]) -> None:
        self.candidates = candidates
        self.dist: dict[str, dict[tuple[str, int], int]] = {name: {} for name in candidates}
        self.margin: dict[tuple[str, int], int] = {}   # top-1 minus top-2, ulps

    def __call__(self, seqs, logits: torch.Tensor) -> None:
        rows = len(seqs)
        top2 = torch.topk(logits, 2 if logits.shape[-1] > 1 else 1, dim=-1).values
        ords = ordinal(top2)
        gap = (ords[:, 0] - ords[:, -1]).tolist()
        best = ords[:, 0]
        idx = [s.num_generated for s in seqs]
        for i, s in enumerate(seqs):
            self.margin[(s.seq_id, idx[i])] = gap[i]
        for name, streams in self.candidates.items():
            want = []
            live = []
            for i, s in enumerate(seqs):
                toks = streams.get(s.seq_id)
                if toks is not None and idx[i] < len(toks):
                    want.append(toks[idx[i]])
                    live.append(i)
            if not live:
                continue
            li = torch.tensor(live, device=logits.device)
            wi = torch.tensor(want, device=logits.device)
            at = ordinal(logits[li, wi].contiguous())
            d = (best[li] - at).tolist()
            for j, i in enumerate(live):
                self.dist[name][(seqs[i].seq_id, idx[i])] = d[j]


def first_divergences(reference: dict[str, list[int]], candidate: dict[str, list[int]],
                      probe: MarginProbe | None = None, name: str | None = None) -> list[dict]:
    """Streams of `candidate` that differ from `reference`: sequence id, first differing
    index, and (with the probe that watched the reference run) the candidate token's
    distance below the reference's maximum logit there and the reference's own
    top-1/top-2 gap, both in ulps."""
    out = []
    for sid, ref in reference.items():
        cand = candidate[sid]
        if cand == ref:
            continue
        n = min(len(ref), len(cand))
        k = next((j for j in range(n) if ref[j] != cand[j]), n)
        row = {"seq": sid, "index": k, "ref_token": ref[k] if k < len(ref) else None,
               "token": cand[k] if k < len(cand) else None}
        if probe is not None:
            row["ulps_below_max"] = probe.dist[name].get((sid, k))
            row["ref_top2_gap_ulps"] = probe.margin.get((sid, k))
        out.append(row)
    return out
