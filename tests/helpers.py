"""Shared checking helpers of the test suite: run the HIP path and the CPU oracle on one input."""
from __future__ import annotations

import sys

import torch

from oracle.brute import decode_fp64
from oracle.ref_torch import ref_gqa_decode_paged, ref_store_kvcache
from tileinfer_amd.kernels.gqa_decode_paged import gqa_decode_paged_fn
from tileinfer_amd.kernels.kvcache_store import store_kvcache
from tileinfer_amd.workloads import PagedStep

# The north star's decode tolerance (bf16 output, fp32 accumulation).
ATOL, RTOL = 2e-2, 1e-2


def say(*args):
    """Print and flush a line naming the case, before the GPU work of a test starts."""
    print(*args, flush=True)
    sys.stdout.flush()


def flat(cache: torch.Tensor) -> torch.Tensor:
    nb, bs, h, d = cache.shape
    return cache.view(nb * bs, h * d)


def gpu_step(step: PagedStep, dev, variant="auto", split_tokens=None, append=True):
    """Copy a CPU step to `dev`, append then decode there; returns (out, k_cache, v_cache) on dev."""
    kc = step.k_cache.to(dev)
    vc = step.v_cache.to(dev)
    if append:
        store_kvcache(step.k_new.to(dev), step.v_new.to(dev), flat(kc), flat(vc),
                      step.slot_mapping.to(dev))
    out = gqa_decode_paged_fn(step.q.to(dev), kc, vc, step.block_table.to(dev),
                              step.seqlen.to(dev), step.page_size, variant=variant,
                              split_tokens=split_tokens)
    return out, kc, vc


def cpu_step(step: PagedStep, append=True):
    """The oracle's append + decode on CPU copies of the step; returns (out, k_cache, v_cache)."""
    kc = step.k_cache.clone()
    vc = step.v_cache.clone()
    if append:
        ref_store_kvcache(step.k_new, step.v_new, flat(kc), flat(vc), step.slot_mapping)
    out = ref_gqa_decode_paged(step.q, kc, vc, step.block_table, step.seqlen, step.page_size)
    return out, kc, vc


def fp64_decode(step: PagedStep, kc: torch.Tensor, vc: torch.Tensor):
    return torch.from_numpy(decode_fp64(step.q.float().numpy(), kc.float().numpy(),
                                        vc.float().numpy(), step.block_table.numpy(),
                                        step.seqlen.numpy(), step.page_size))


def assert_decode_close(out: torch.Tensor, ref: torch.Tensor, atol=ATOL, rtol=RTOL):
    torch.testing.assert_close(out.detach().float().cpu(), ref.float().cpu(), atol=atol, rtol=rtol)


def bits(t: torch.Tensor) -> torch.Tensor:
    """16-bit payload of a bf16/fp16 tensor, for bit-exact comparisons."""
    return t.contiguous().view(torch.int16)
