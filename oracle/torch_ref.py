"""Torch fp32 restatement of the reference's golden ``run()`` -- TEST AND
BASELINE INFRASTRUCTURE ONLY (imported by ``tests/`` and by the
``cpu_baseline`` leg of ``bench.py``; the product path never imports it).

``run_fp32`` follows ``solution/triton/indexer_kernel.py:436-497`` step for
step on the CPU: the whole paged cache is converted to fp32 first
(``:457-459``), then a per-token loop gathers the valid slots (``:467-481``),
forms the scaled logits (``:486-487``), the base-2 log-sum-exp (``:490``) and
``softmax(logits) @ Kc`` rounded to bf16 (``:493-495``); a row without valid
slots keeps a zero output and ``lse = -inf`` (``:463-475``).  The constant
asserts of ``:444-448`` (H=16, page_size=64, topk=2048) are left out so every
configuration runs, and ``math`` is imported (``:490`` uses it without the
import the reference file lacks).  It is pinned against the fp64 C oracle in
``tests/test_oracle.py`` (reference checker tolerances).
"""
from __future__ import annotations

import math

import torch


@torch.no_grad()
def run_fp32(q_nope: torch.Tensor, q_pe: torch.Tensor, ckv_cache: torch.Tensor,
             kpe_cache: torch.Tensor, sparse_indices: torch.Tensor, sm_scale: float):
    """``(output [T,H,512] bf16, lse [T,H] fp32 base 2)`` on the CPU."""
    T, H, dc = q_nope.shape
    dp = q_pe.shape[-1]
    kc_all = ckv_cache.reshape(-1, dc).to(torch.float32)
    kp_all = kpe_cache.reshape(-1, dp).to(torch.float32)
    output = torch.zeros((T, H, dc), dtype=torch.bfloat16)
    lse = torch.full((T, H), -float("inf"), dtype=torch.float32)
    inv_ln2 = 1.0 / math.log(2.0)
    for t in range(T):
        idx = sparse_indices[t]
        valid = idx[idx != -1]
        if valid.numel() == 0:
            continue
        tok = valid.to(torch.long)
        kc = kc_all[tok]
        kp = kp_all[tok]
        qn = q_nope[t].to(torch.float32)
        qp = q_pe[t].to(torch.float32)
        logits = (qn @ kc.T + qp @ kp.T) * sm_scale
        lse[t] = torch.logsumexp(logits, dim=-1) * inv_ln2
        output[t] = (torch.softmax(logits, dim=-1) @ kc).to(torch.bfloat16)
    return output, lse
