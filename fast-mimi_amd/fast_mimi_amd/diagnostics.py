"""Near-tie margins of RVQ codes (reported beside throughput).

For each codebook step the quantizer picks the entry nearest to the residual
(``MimiEuclideanCodebook.quantize``, reference ``model.py:2277-2291``).  Two
implementations that sum the 258-term mm-form distance in different orders
can only disagree where the best two entries are within a few FP32 ulps of
|x|^2 + |e|^2.  ``code_margins`` re-evaluates, in float64 on the device, the
distances along the code chain the GPU produced and reports the smallest
relative gap between the best and second-best entry, how many rows fall
below a threshold, and whether each GPU code is the float64 nearest entry.
"""

from __future__ import annotations

import torch


@torch.inference_mode()
def code_margins(model, audio: torch.Tensor, codes: torch.Tensor, near: float = 1e-6) -> dict:
    """audio [B, 1, S] on the model's device; codes [B, nq, T] from the model."""
    rt = model.runtime()
    cfg = model.config
    B, nq, T = codes.shape
    with torch.cuda.device(model.device):
        h, b, t = rt.embeddings(audio.to(model.device, torch.float32).contiguous())
        proj = rt.quantizer_inputs(h, b, t).double()
    assert b == B and t == T, (b, t, B, T)
    vq = rt.vq
    n_sem = min(cfg.num_semantic_quantizers, nq)
    flat = codes.to(model.device).transpose(0, 1).reshape(nq, B * T)
    min_gap, rows_near, not_nearest = float("inf"), 0, 0
    for first, count, col in ((0, n_sem, 0), (n_sem, nq - n_sem, vq)):
        residual = proj[:, col:col + vq].clone()
        for j in range(first, first + count):
            e = rt.embeds[j].double()
            en = (e * e).sum(-1)
            xn = (residual * residual).sum(-1, keepdim=True)
            d2 = xn + en[None] - 2.0 * residual @ e.T
            top = torch.topk(d2, 2, dim=-1, largest=False)
            gap = (top.values[:, 1] - top.values[:, 0]) / (xn[:, 0] + en[top.indices[:, 0]])
            min_gap = min(min_gap, float(gap.min()))
            rows_near += int((gap < near).sum())
            not_nearest += int((top.indices[:, 0] != flat[j]).sum())
            residual = residual - e[flat[j]]
    return {"min_top2_rel_gap": min_gap, f"rows_gap_below_{near:.0e}": rows_near,
            "codes_not_fp64_nearest": not_nearest, "code_rows": int(B * T * nq)}
