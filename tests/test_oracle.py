"""Pins the CPU oracle: closed forms, invariants, an independent scalar spelling, the committed
golden fixtures, and planted mistakes that the checks must catch. CPU only."""
import hashlib
import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle.brute import decode_fp64, decode_loop_fp64, store_np
from oracle.ref_torch import ref_gqa_decode_paged, ref_store_kvcache
from tileinfer_amd.workloads import config1, make_step

GOLDEN = Path(__file__).resolve().parent / "golden"


def _u16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


# ----------------------------------------------------------------------------- append


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_store_oracle_equals_closed_form(dtype):
    g = torch.Generator().manual_seed(1)
    n, h, d, slots_n = 37, 4, 64, 300
    key = torch.randn(n, h, d, generator=g).to(dtype)
    value = torch.randn(n, h, d, generator=g).to(dtype)
    slots = torch.randperm(slots_n, generator=g)[:n].to(torch.int32)
    slots[::7] = -1
    kc = torch.randn(slots_n, h * d, generator=g).to(dtype)
    vc = torch.randn(slots_n, h * d, generator=g).to(dtype)
    k_exp, v_exp = store_np(_u16(key), _u16(value), _u16(kc), _u16(vc), slots.numpy())
    ref_store_kvcache(key, value, kc, vc, slots)
    assert np.array_equal(_u16(kc), k_exp) and np.array_equal(_u16(vc), v_exp)
    # Rows with slot >= 0 hold the new rows; all others equal the pre-append cache.
    live = slots.numpy() >= 0
    assert np.array_equal(k_exp[slots.numpy()[live]], _u16(key).reshape(n, -1)[live])


def test_store_oracle_noops():
    kc = torch.randn(10, 8).to(torch.bfloat16)
    vc = torch.randn(10, 8).to(torch.bfloat16)
    k0, v0 = kc.clone(), vc.clone()
    ref_store_kvcache(torch.zeros(0, 2, 4, dtype=torch.bfloat16),
                      torch.zeros(0, 2, 4, dtype=torch.bfloat16), kc, vc,
                      torch.zeros(0, dtype=torch.int32))
    ref_store_kvcache(torch.ones(3, 2, 4, dtype=torch.bfloat16),
                      torch.ones(3, 2, 4, dtype=torch.bfloat16), kc, vc,
                      torch.full((3,), -1, dtype=torch.int32))
    assert torch.equal(kc, k0) and torch.equal(vc, v0)


# ----------------------------------------------------------------------------- decode


def _tiny(seed=0, ctx=(0, 1, 5, 9, 16), bs=4, hq=4, hkv=2, d=8, pool=40):
    g = torch.Generator().manual_seed(seed)
    need = [(c + bs - 1) // bs for c in ctx]
    perm = torch.randperm(pool, generator=g)
    w = max(max(need), 1)
    table = torch.full((len(ctx), w), -1, dtype=torch.int32)
    off = 0
    for i, n in enumerate(need):
        table[i, :n] = perm[off:off + n].to(torch.int32)
        off += n
    q = torch.randn(len(ctx), hq, d, generator=g)
    kc = torch.randn(pool, bs, hkv, d, generator=g)
    vc = torch.randn(pool, bs, hkv, d, generator=g)
    return q, kc, vc, table, torch.tensor(ctx, dtype=torch.int32), bs


def test_fp64_vectorised_equals_scalar_loops():
    q, kc, vc, table, seq, bs = _tiny()
    vec = decode_fp64(q.numpy(), kc.numpy(), vc.numpy(), table.numpy(), seq.numpy(), bs)
    loop = np.array(decode_loop_fp64(q.tolist(), kc.tolist(), vc.tolist(), table.tolist(),
                                     seq.tolist(), bs))
    np.testing.assert_allclose(vec, loop, rtol=1e-12, atol=1e-12)


def test_fp64_closed_forms():
    q, kc, vc, table, seq, bs = _tiny(ctx=(1, 7))
    out = decode_fp64(q.numpy(), kc.numpy(), vc.numpy(), table.numpy(), seq.numpy(), bs)
    blk = int(table[0, 0])
    # ctx 1: the row of V of the mapped KV head (head h reads KV head h // 2).
    for h in range(4):
        np.testing.assert_allclose(out[0, h], vc[blk, 0, h // 2].double().numpy(), rtol=1e-12)
    # q = 0: equal scores, the output is the mean of V over the context.
    out0 = decode_fp64(np.zeros_like(q.numpy()), kc.numpy(), vc.numpy(), table.numpy(),
                       seq.numpy(), bs)
    rows = [int(table[1, p // bs]) * bs + p % bs for p in range(7)]
    vflat = vc.double().reshape(-1, 2, 8).numpy()
    np.testing.assert_allclose(out0[1, 3], vflat[rows, 1].mean(0), rtol=1e-12)
    # Hand-computed two-token case: scores 0 and ln 3 give weights 1/4 and 3/4.
    d = 4
    qh = np.zeros((1, 1, d))
    qh[0, 0, 0] = math.sqrt(d)
    kh = np.zeros((1, 2, 1, d))
    kh[0, 1, 0, 0] = math.log(3.0)
    vh = np.zeros((1, 2, 1, d))
    vh[0, 0, 0, 1] = 4.0
    vh[0, 1, 0, 2] = 8.0
    o = decode_fp64(qh, kh, vh, np.array([[0]]), np.array([2]), 2)
    np.testing.assert_allclose(o[0, 0], [0.0, 1.0, 6.0, 0.0], rtol=1e-12, atol=1e-15)


@pytest.mark.parametrize("scale", [1.0 / 16, 1.0])
def test_ref_recipe_within_tolerance_of_fp64(scale):
    step = make_step([1, 17, 300, 1000], pool=100, seed=5, value_scale=scale)
    ref = ref_gqa_decode_paged(step.q, step.k_cache, step.v_cache, step.block_table,
                               step.seqlen, 16)
    exact = decode_fp64(step.q.float().numpy(), step.k_cache.float().numpy(),
                        step.v_cache.float().numpy(), step.block_table.numpy(),
                        step.seqlen.numpy(), 16)
    np.testing.assert_allclose(ref.float().numpy(), exact, atol=2e-2, rtol=1e-2)


def test_ref_recipe_bitwise_invariants():
    step = make_step([40, 200, 129], pool=40, seed=6)
    base = ref_gqa_decode_paged(step.q, step.k_cache, step.v_cache, step.block_table,
                                step.seqlen, 16)
    # Renaming physical blocks changes nothing.
    perm = torch.randperm(40, generator=torch.Generator().manual_seed(1))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(40)
    tbl = step.block_table.clone()
    live = tbl >= 0
    tbl[live] = perm[tbl[live].long()].to(torch.int32)
    out = ref_gqa_decode_paged(step.q, step.k_cache[inv], step.v_cache[inv], tbl, step.seqlen, 16)
    assert torch.equal(out, base)
    # Extra -1 columns past each sequence are never read.
    wide = torch.full((3, 40), -1, dtype=torch.int32)
    wide[:, :step.block_table.shape[1]] = step.block_table
    assert torch.equal(ref_gqa_decode_paged(step.q, step.k_cache, step.v_cache, wide,
                                            step.seqlen, 16), base)
    # ctx 0 gives zeros.
    z = ref_gqa_decode_paged(step.q[:1], step.k_cache, step.v_cache, step.block_table[:1],
                             torch.zeros(1, dtype=torch.int32), 16)
    assert not bool(z.any())


def test_ref_recipe_shared_vs_private_prefix():
    # Two sequences: shared tables alias the same 3 prefix blocks; private copies duplicate them.
    g = torch.Generator().manual_seed(3)
    kc = torch.randn(10, 16, 4, 256, generator=g).to(torch.bfloat16)
    vc = torch.randn(10, 16, 4, 256, generator=g).to(torch.bfloat16)
    q = torch.randn(2, 24, 256, generator=g).to(torch.bfloat16)
    seq = torch.tensor([60, 58], dtype=torch.int32)
    shared = torch.tensor([[0, 1, 2, 3], [0, 1, 2, 4]], dtype=torch.int32)
    kp, vp = kc.clone(), vc.clone()
    kp[5:8], vp[5:8] = kc[0:3], vc[0:3]
    private = torch.tensor([[0, 1, 2, 3], [5, 6, 7, 4]], dtype=torch.int32)
    assert torch.equal(ref_gqa_decode_paged(q, kc, vc, shared, seq),
                       ref_gqa_decode_paged(q, kp, vp, private, seq))


def test_ref_recipe_head_mapping():
    """Query head h reads KV head h // (Hq/Hkv): with a distinct constant V per KV head the
    output of head h is that head's constant (exact for ctx 1)."""
    step = make_step([1], pool=2, seed=2)
    vc = torch.zeros_like(step.v_cache)
    for kvh in range(4):
        vc[:, :, kvh, :] = float(kvh + 1)
    out = ref_gqa_decode_paged(step.q, step.k_cache, vc, step.block_table, step.seqlen)
    for h in range(24):
        assert bool((out[0, h] == float(h // 6 + 1)).all())


def _mutant_head_mod(q, kc, vc, bt, seq, ps=16):
    """Planted mistake: query head h reads KV head h % Hkv instead of h // G."""
    b_sz, h_q, d = q.shape
    h_kv = kc.shape[2]
    out = torch.zeros_like(q)
    for b in range(b_sz):
        n = int(seq[b])
        pages = bt[b, :(n + ps - 1) // ps].long()
        k = kc[pages].reshape(-1, h_kv, d)[:n]
        v = vc[pages].reshape(-1, h_kv, d)[:n]
        for h in range(h_q):
            s = (q[b, h].float() @ k[:, h % h_kv].float().T) * d ** -0.5
            out[b, h] = (torch.softmax(s, -1) @ v[:, h % h_kv].float()).to(q.dtype)
    return out


def _mutant_no_scale(q, kc, vc, bt, seq, ps=16):
    """Planted mistake: the D^-1/2 score scale is dropped."""
    return ref_gqa_decode_paged(q * 16.0, kc, vc, bt, seq, ps)


def _mutant_off_by_one(q, kc, vc, bt, seq, ps=16):
    """Planted mistake: the newest token (position ctx-1) is left out of the context."""
    return ref_gqa_decode_paged(q, kc, vc, bt, (seq - 1).clamp(min=0), ps)


@pytest.mark.parametrize("mutant", [_mutant_head_mod, _mutant_no_scale, _mutant_off_by_one])
def test_checks_catch_planted_mistakes(mutant):
    step = make_step([3, 50, 333], pool=40, seed=7)
    args = (step.q, step.k_cache, step.v_cache, step.block_table, step.seqlen, 16)
    exact = decode_fp64(step.q.float().numpy(), step.k_cache.float().numpy(),
                        step.v_cache.float().numpy(), step.block_table.numpy(),
                        step.seqlen.numpy(), 16)
    np.testing.assert_allclose(ref_gqa_decode_paged(*args).float().numpy(), exact,
                               atol=2e-2, rtol=1e-2)
    with pytest.raises(AssertionError):
        np.testing.assert_allclose(mutant(*args).float().numpy(), exact, atol=2e-2, rtol=1e-2)


# ----------------------------------------------------------------------------- golden fixtures


@pytest.mark.parametrize("ctx", [512, 513])
def test_golden_config1(ctx):
    meta = json.loads((GOLDEN / f"config1_ctx{ctx}.json").read_text())
    step = config1(seed=meta["seed"], ctx=ctx)
    for name, want in meta["inputs_sha256"].items():
        t = getattr(step, name).contiguous().view(-1).view(torch.uint8).numpy().tobytes()
        assert hashlib.sha256(t).hexdigest() == want, f"input {name} drifted (generator change?)"
    assert int(step.slot_mapping[0]) == meta["slot"]
    kc, vc = step.k_cache.clone(), step.v_cache.clone()
    ref_store_kvcache(step.k_new, step.v_new, kc.view(-1, 1024), vc.view(-1, 1024),
                      step.slot_mapping)
    out = ref_gqa_decode_paged(step.q, kc, vc, step.block_table, step.seqlen, 16)
    gold = np.load(GOLDEN / f"config1_ctx{ctx}_out.npy")
    assert np.array_equal(_u16(out).reshape(24, 256), gold)
    exact = decode_fp64(step.q.float().numpy(), kc.float().numpy(), vc.float().numpy(),
                        step.block_table.numpy(), step.seqlen.numpy(), 16)
    np.testing.assert_allclose(out.float().numpy(), exact, atol=2e-2, rtol=1e-2)
