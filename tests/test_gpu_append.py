"""Bit-exact parity of the HIP append (ti_kv_append) with the oracle and the append's closed form."""
import pytest
import torch

from helpers import bits, cpu_step, flat, say
from oracle.ref_torch import ref_store_kvcache
from tileinfer_amd.kernels.kvcache_store import store_kvcache
from tileinfer_amd.workloads import config1, config2, config4

pytestmark = pytest.mark.gpu


def _append_gpu(key, value, kc, vc, slots, dev):
    kd, vd = kc.to(dev), vc.to(dev)
    store_kvcache(key.to(dev), value.to(dev), kd, vd, slots.to(dev))
    return kd.cpu(), vd.cpu()


@pytest.mark.parametrize("cfg", ["config1", "config2"])
def test_append_matches_oracle(cfg, dev):
    step = {"config1": config1, "config2": config2}[cfg]()
    say(f"append {cfg}: N={step.slot_mapping.numel()} slots")
    _, k_ref, v_ref = cpu_step(step)  # oracle append (decode output unused)
    kd, vd = _append_gpu(step.k_new, step.v_new, flat(step.k_cache), flat(step.v_cache),
                         step.slot_mapping, dev)
    assert torch.equal(bits(kd), bits(flat(k_ref)))
    assert torch.equal(bits(vd), bits(flat(v_ref)))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_append_reference_selftest_shape(dtype, dev):
    # kernels/kvcache_store.py:88-99: N=8, 4 heads x 128, 1024 slots, every 10th slot -1
    # (unique slots here: duplicates are unsupported).
    say(f"append selftest shape {dtype}")
    g = torch.Generator().manual_seed(42)
    n, h, d, slots_n = 8, 4, 128, 1024
    key = torch.randn(n, h, d, generator=g).to(dtype)
    value = torch.randn(n, h, d, generator=g).to(dtype)
    slots = torch.randperm(slots_n, generator=g)[:n].to(torch.int32)
    slots[::10] = -1
    kc = torch.zeros(slots_n, h * d, dtype=dtype)
    vc = torch.zeros(slots_n, h * d, dtype=dtype)
    k_ref, v_ref = kc.clone(), vc.clone()
    ref_store_kvcache(key, value, k_ref, v_ref, slots)
    kd, vd = _append_gpu(key, value, kc, vc, slots, dev)
    assert torch.equal(bits(kd), bits(k_ref)) and torch.equal(bits(vd), bits(v_ref))


def test_append_config4_mixed_step(dev):
    """2,048-token chunk over 128 non-contiguous blocks + 32 decode tokens in one call (N=2,080)."""
    step, chunk_slots = config4(device=dev)
    say(f"append config4: N={chunk_slots.numel() + step.slot_mapping.numel()}")
    key = torch.cat([step.meta["chunk_k"], step.k_new])
    value = torch.cat([step.meta["chunk_v"], step.v_new])
    slots = torch.cat([chunk_slots, step.slot_mapping])
    kd = step.k_cache.to(dev)
    vd = step.v_cache.to(dev)
    before_k, before_v = kd.clone(), vd.clone()
    store_kvcache(key.to(dev), value.to(dev), flat(kd), flat(vd), slots.to(dev))
    s = slots.to(dev).long()
    # Closed form: written rows equal the new rows, every other row is untouched.
    assert torch.equal(bits(flat(kd)[s]), bits(key.to(dev).reshape(len(s), -1)))
    assert torch.equal(bits(flat(vd)[s]), bits(value.to(dev).reshape(len(s), -1)))
    keep = torch.ones(flat(kd).shape[0], dtype=torch.bool, device=dev)
    keep[s] = False
    assert torch.equal(bits(flat(kd)[keep]), bits(flat(before_k)[keep]))
    assert torch.equal(bits(flat(vd)[keep]), bits(flat(before_v)[keep]))


def test_append_edge_cases(dev):
    say("append edge cases")
    g = torch.Generator().manual_seed(7)
    n, h, d, slots_n = 6, 4, 256, 64
    key = torch.randn(n, h, d, generator=g).to(torch.bfloat16)
    value = torch.randn(n, h, d, generator=g).to(torch.bfloat16)
    kc = torch.randn(slots_n, h * d, generator=g).to(torch.bfloat16)
    vc = torch.randn(slots_n, h * d, generator=g).to(torch.bfloat16)
    # N = 0: no-op.
    kd, vd = _append_gpu(key[:0], value[:0], kc, vc, torch.zeros(0, dtype=torch.int32), dev)
    assert torch.equal(bits(kd), bits(kc)) and torch.equal(bits(vd), bits(vc))
    # All slots -1: no-op.
    kd, vd = _append_gpu(key, value, kc, vc, torch.full((n,), -1, dtype=torch.int32), dev)
    assert torch.equal(bits(kd), bits(kc)) and torch.equal(bits(vd), bits(vc))
    # A slot at/after num_slots is skipped; the others are written.
    slots = torch.tensor([3, slots_n, 9, -1, slots_n + 100, 0], dtype=torch.int32)
    ok = slots.clone()
    ok[(ok >= slots_n)] = -1
    k_ref, v_ref = kc.clone(), vc.clone()
    ref_store_kvcache(key, value, k_ref, v_ref, ok)
    kd, vd = _append_gpu(key, value, kc, vc, slots, dev)
    assert torch.equal(bits(kd), bits(k_ref)) and torch.equal(bits(vd), bits(v_ref))


def test_append_strided_key(dev):
    """k.squeeze(2) of a [B, H, 1, D] projection and a transposed prefill view both work."""
    say("append strided key")
    g = torch.Generator().manual_seed(11)
    b, h, d, slots_n = 5, 4, 256, 80
    k4 = torch.randn(b, h, 3, d, generator=g).to(torch.bfloat16)[:, :, 1:2, :]
    key = k4.squeeze(2)               # non-contiguous [B, H, D]
    value = torch.randn(h, b, d, generator=g).to(torch.bfloat16).transpose(0, 1)
    slots = torch.randperm(slots_n, generator=g)[:b].to(torch.int32)
    kc = torch.zeros(slots_n, h * d, dtype=torch.bfloat16)
    vc = torch.zeros(slots_n, h * d, dtype=torch.bfloat16)
    k_ref, v_ref = kc.clone(), vc.clone()
    ref_store_kvcache(key, value, k_ref, v_ref, slots)
    kd, vd = _append_gpu(key, value, kc, vc, slots, dev)
    assert torch.equal(bits(kd), bits(k_ref)) and torch.equal(bits(vd), bits(v_ref))


def test_append_bulk_65536(dev):
    say("append bulk N=65536")
    n, h, d = 65536, 4, 256
    slots_n = 2 * n
    gen = torch.Generator(device=dev).manual_seed(5)
    key = torch.randn(n, h, d, generator=gen, device=dev).to(torch.bfloat16)
    value = torch.randn(n, h, d, generator=gen, device=dev).to(torch.bfloat16)
    slots = torch.randperm(slots_n, generator=gen, device=dev)[:n].to(torch.int32)
    kc = torch.zeros(slots_n, h * d, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros(slots_n, h * d, dtype=torch.bfloat16, device=dev)
    store_kvcache(key, value, kc, vc, slots)
    s = slots.long()
    assert torch.equal(bits(kc[s]), bits(key.reshape(n, -1)))
    assert torch.equal(bits(vc[s]), bits(value.reshape(n, -1)))
    keep = torch.ones(slots_n, dtype=torch.bool, device=dev)
    keep[s] = False
    assert not bool((kc[keep].view(torch.int16) != 0).any())
    assert not bool((vc[keep].view(torch.int16) != 0).any())
