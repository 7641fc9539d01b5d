"""RVQ code parity with near-tie certification.

Torch's CPU cdist and the GPU distance GEMM sum the same 258 products in
different orders, so their FP32 distances differ by a few ulps of
|x|^2 + |e|^2 (the magnitude the mm-form cancels from; one FP32 ulp of it is
~6e-8 relative).  Codes can only legitimately differ where the two best
candidates are that close.

``check_codes`` compares GPU codes with the reference's.  Where exactness is
required (``allow=None``) any difference fails.  Otherwise each differing
(row, codebook) is re-evaluated in float64 on the reference's residual and
*certified* only when the float64 distance gap is below ``NEAR_TIE_TOL`` of
|x|^2 + |e|^2; the chain of that row is then restarted on the GPU from the
reference's residual after the near-tie codebook, so every later codebook of
the row is still compared.  The count of certified near-ties and the worst gap
must stay within ``allow = (max_rows, max_gap)``.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch
import torch.nn.functional as F

# ~16 FP32 ulps of |x|^2 + |e|^2: the summation-order noise of a 258-term
# mm-form distance, well below any gap a wrong product or index would leave.
NEAR_TIE_TOL = 1e-6


@dataclass
class CodeReport:
    near_ties: list = field(default_factory=list)  # (b, j, t, ref, gpu, rel_gap)

    @property
    def count(self) -> int:
        return len(self.near_ties)

    @property
    def worst_gap(self) -> float:
        return max((r[-1] for r in self.near_ties), default=0.0)

    def summary(self) -> str:
        return f"{self.count} certified near-tie codes (worst relative gap {self.worst_gap:.2e})"


def first_divergence(got: torch.Tensor, want: torch.Tensor):
    """codes [B, nq, T] -> list of (b, j, t) at the first differing codebook."""
    diff = got != want
    out = []
    for b, t in zip(*torch.nonzero(diff.any(1), as_tuple=True)):
        j = int(torch.nonzero(diff[b, :, t])[0])
        out.append((int(b), j, int(t)))
    return out


def relative_gap(x: torch.Tensor, e: torch.Tensor, ia: int, ib: int) -> float:
    """float64 |d(x, e_ia) - d(x, e_ib)| (squared distances) over |x|^2 + max |e|^2."""
    x, e = x.double(), e.double()
    da = ((x - e[ia]) ** 2).sum()
    db = ((x - e[ib]) ** 2).sum()
    scale = (x * x).sum() + max(float((e[ia] ** 2).sum()), float((e[ib] ** 2).sum()))
    return float((da - db).abs() / scale)


def check_codes(got, want, rows_per_step, embeds, n_semantic, rerun=None, allow=None,
                tol=NEAR_TIE_TOL) -> CodeReport:
    """got / want: codes [B, nq, T]; rows_per_step[j]: the reference's residual
    rows [B*T, D] entering codebook j; embeds[j]: codebook j.  ``rerun(x, j0,
    count)`` runs the GPU chain of codebooks j0 .. j0+count-1 on rows x [R, D]
    and returns codes [count, R].  Raises AssertionError on any uncertified or
    out-of-budget difference."""
    assert got.shape == want.shape, (got.shape, want.shape)
    report = CodeReport()
    B, nq, T = want.shape
    pending = first_divergence(got, want)
    if pending and allow is None:
        b, j, t = pending[0]
        raise AssertionError(
            f"{len(pending)} code rows differ from the reference (bit-exact required); first at "
            f"batch {b} codebook {j} frame {t}: ref {int(want[b, j, t])} gpu {int(got[b, j, t])}")
    got = got.clone()  # rows re-run from the reference's residual are written back here
    while pending:
        nxt = []
        for b, j, t in pending:
            ia, ib = int(want[b, j, t]), int(got[b, j, t])
            rel = relative_gap(rows_per_step[j][b * T + t], embeds[j], ia, ib)
            assert rel <= tol, (
                f"uncertified code mismatch at batch {b} codebook {j} frame {t}: "
                f"ref {ia} gpu {ib}, relative gap {rel:.3e} > {tol:.0e}")
            report.near_ties.append((b, j, t, ia, ib, rel))
            end = n_semantic if j < n_semantic else nq
            if j + 1 >= end:
                continue
            assert rerun is not None, "a near-tie inside a chain needs the GPU re-run to compare the rest"
            x = rows_per_step[j + 1][b * T + t][None].contiguous()
            got[b, j + 1:end, t] = rerun(x, j + 1, end - j - 1)[:, 0].cpu()
            diff = torch.nonzero(got[b, j + 1:end, t] != want[b, j + 1:end, t])
            if len(diff):
                nxt.append((b, j + 1 + int(diff[0]), t))
        pending = nxt
    if allow is not None:
        max_rows, max_gap = allow
        assert report.count <= max_rows and report.worst_gap <= max_gap, (
            f"{report.summary()} exceeds the recorded bound ({max_rows} rows, gap {max_gap:.1e})")
    return report


def reference_rvq_rows(x: torch.Tensor, embeds, codes_flat: torch.Tensor):
    """Residual rows entering each codebook along the reference's code chain.
    x [M, D]; codes_flat [nq, M]."""
    rows = []
    residual = x.clone()
    for j, e in enumerate(embeds):
        rows.append(residual)
        residual = residual - F.embedding(codes_flat[j], e)
    return rows
