"""Near-tie certification of RVQ code mismatches.

Torch's CPU cdist and the GPU distance GEMM sum the same 258 products in
different orders, so their FP32 distances differ by up to a few ulps of
|x|^2 + |e|^2 (the magnitude the mm-form cancels from).  Codes can only
legitimately differ where the two best candidates are that close.  For every
row, the first codebook at which the two code chains differ is re-evaluated in
float64 on the identical residual; the mismatch is *certified* when the float64
distance gap is below ``tol * (|x|^2 + |e|^2)``.  Later codebooks of a row
whose chain already diverged are not compared (their residuals differ).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def first_divergence(got: torch.Tensor, want: torch.Tensor):
    """codes [B, nq, T] -> list of (b, j, t) at the first differing codebook."""
    diff = got != want
    out = []
    for b, t in zip(*torch.nonzero(diff.any(1), as_tuple=True)):
        j = int(torch.nonzero(diff[b, :, t])[0])
        out.append((int(b), j, int(t)))
    return out


def certify(rows_per_step, embeds, got, want, tol=1e-5):
    """rows_per_step[j]: the reference's residual rows [B*T, D] entering codebook
    j (float32); embeds[j]: codebook j.  Returns (n_mismatch_rows, worst_rel_gap);
    raises AssertionError on an uncertified mismatch."""
    B, nq, T = want.shape
    worst = 0.0
    div = first_divergence(got, want)
    for b, j, t in div:
        x = rows_per_step[j][b * T + t].double()
        e = embeds[j].double()
        ia, ib = int(want[b, j, t]), int(got[b, j, t])
        da = ((x - e[ia]) ** 2).sum()
        db = ((x - e[ib]) ** 2).sum()
        scale = (x * x).sum() + max(float((e[ia] ** 2).sum()), float((e[ib] ** 2).sum()))
        rel = float((da - db).abs() / scale)
        worst = max(worst, rel)
        assert rel <= tol, (
            f"uncertified code mismatch at batch {b} codebook {j} frame {t}: "
            f"ref {ia} gpu {ib}, relative gap {rel:.3e}")
    return len(div), worst


def reference_rvq_rows(x: torch.Tensor, embeds, codes_flat: torch.Tensor):
    """Residual rows entering each codebook along the reference's code chain.
    x [M, D]; codes_flat [nq, M]."""
    rows = []
    residual = x.clone()
    for j, e in enumerate(embeds):
        rows.append(residual)
        residual = residual - F.embedding(codes_flat[j], e)
    return rows
