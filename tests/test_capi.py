"""The C-ABI library loads, exports every symbol include/tileinfer_amd.h declares, and rejects bad
arguments before touching a device (CPU only: no kernel is launched here)."""
import ctypes
import re
from pathlib import Path

import pytest
import torch

from tileinfer_amd import _lib
from tileinfer_amd.kernels.gqa_decode_paged import gqa_decode_paged_fn
from tileinfer_amd.kernels.gqa_prefill_paged import gqa_prefill_paged_fn
from tileinfer_amd.kernels.kvcache_store import store_kvcache

HEADER = Path(__file__).resolve().parents[1] / "include" / "tileinfer_amd.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(ti_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_functions()
    assert names == sorted(_lib.SIGNATURES), "ctypes table out of sync with the header"
    for name in names:
        assert hasattr(lib, name), f"{name} not exported"
    assert lib.ti_abi_version() == _lib.ABI_VERSION


def test_header_codes_match_binding():
    text = HEADER.read_text()
    for name in ("TI_OK", "TI_EINVAL", "TI_ELAUNCH", "TI_EUNSUPPORTED", "TI_DTYPE_BF16",
                 "TI_DTYPE_F16", "TI_DECODE_AUTO", "TI_DECODE_MFMA", "TI_DECODE_SCALAR",
                 "TI_DECODE_REUSE_KV", "TI_DECODE_STREAM_KV"):
        m = re.search(rf"#define {name} (0x[0-9a-fA-F]+|\d+)", text)
        assert m and int(m.group(1), 0) == getattr(_lib, name), name


def _plan(*args):
    lib = _lib.load()
    s, m, w = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int64()
    rc = lib.ti_gqa_decode_plan(*args, ctypes.byref(s), ctypes.byref(m), ctypes.byref(w))
    return rc, s.value, m.value, w.value


def test_decode_plan_sizes():
    # Config 3 with 2048-token partitions: 16 partitions, fp32 partials (o + m,l) per q-head.
    rc, split, ms, ws = _plan(64, 24, 4, 256, 16, 2048, 2048)
    assert (rc, split, ms, ws) == (0, 2048, 16, 64 * 24 * 16 * (256 + 2) * 4)
    # A bound that fits one partition needs no workspace.
    assert _plan(8, 24, 4, 256, 16, 64, 2048)[1:] == (2048, 1, 0)


def test_balanced_plan_one_wave_per_simd_in_whole_rounds():
    """The balanced decode plan (no split requested; this container has no device, so the plan
    takes MI355X's 256 CUs) gives every SIMD one KV-head wave per round: 1,024 / H_kv runs per
    KV-head group, whatever the workgroup size. When the block ids one run may stage (1,023
    16-token tiles at page size 16) force more runs, it takes whole extra rounds, never a partial
    one: a partial round runs alone after the others and nearly doubles the time."""
    for hkv, hq, d in ((4, 24, 256), (8, 32, 128), (2, 16, 128), (1, 8, 128), (2, 12, 256)):
        rc, split, wgs, ws = _plan(64, hq, hkv, d, 16, 512, 0)  # 64 x 8k: one round
        assert (rc, split, wgs) == (0, 0, 1024 // hkv)
        assert ws >= wgs * 2 * hq * (d + 2) * 4
    # 64 x 32k at 8 KV heads: 131,072 tiles in runs of at most 1,023 need 129 runs per group, one
    # more than a round holds (128), so two whole rounds (256 runs), not 129.
    assert _plan(64, 32, 8, 128, 16, 2048, 0)[2] == 256
    # At 4 KV heads the same batch fits one round (256 runs of 512 tiles).
    assert _plan(64, 24, 4, 256, 16, 2048, 0)[2] == 256


def test_short_bounds_take_fixed_partitions():
    """With no split requested, context bounds of at most 1,024 tokens whose smallest fixed
    partitions fit one round of workgroups take that fixed split (lcm(32, page) tokens); longer
    bounds, or batches whose partitions exceed one round, stay balanced. Bounds of at most 128
    tokens whose (sequence, KV head) pairs fit one round take one workgroup per pair instead
    (reported as split 0 over 0 runs). The workspace covers every plan of the bounds (the
    balanced one is the largest here)."""
    ws_balanced = 256 * 2 * 24 * 258 * 4 + 256
    assert _plan(1, 24, 4, 256, 16, 32, 0) == (0, 32, 16, ws_balanced)      # config 1: 512 tokens
    assert _plan(1, 24, 4, 256, 16, 64, 0)[1:3] == (32, 32)                  # 1,024 tokens
    assert _plan(1, 24, 4, 256, 16, 65, 0)[1:3] == (0, 256)                  # 1,040: balanced
    assert _plan(16, 24, 4, 256, 16, 32, 0)[1:3] == (32, 16)                 # 256 workgroups
    assert _plan(17, 24, 4, 256, 16, 32, 0)[1:3] == (0, 256)                 # 272: balanced
    assert _plan(5, 24, 4, 256, 8, 64, 0)[1:3] == (32, 16)                   # page 8, 512 tokens
    assert _plan(5, 24, 4, 256, 64, 8, 0)[1:3] == (64, 8)                    # page 64: 512 tokens
    assert _plan(16, 32, 8, 128, 16, 16, 0)[1:3] == (32, 8)                  # 2 KV-head groups
    assert _plan(17, 32, 8, 128, 16, 16, 0)[1:3] == (0, 128)
    # One workgroup per (sequence, KV head): up to 128 tokens, up to 256 pairs.
    assert _plan(1, 24, 4, 256, 16, 8, 0)[1:3] == (0, 0)                     # 128 tokens
    assert _plan(1, 24, 4, 256, 16, 9, 0)[1:3] == (32, 5)                    # 144: fixed
    assert _plan(64, 24, 4, 256, 16, 8, 0)[1:3] == (0, 0)                    # 256 pairs
    assert _plan(65, 24, 4, 256, 16, 8, 0)[1:3] == (0, 256)                  # 260 pairs: balanced
    assert _plan(32, 32, 8, 128, 16, 4, 0)[1:3] == (0, 0)
    assert _plan(1, 24, 4, 256, 8, 16, 0)[1:3] == (0, 0)                     # page 8, 128 tokens
    # A requested split is kept as it is.
    assert _plan(1, 24, 4, 256, 16, 32, 256)[1:3] == (256, 2)
    assert _plan(1, 24, 4, 256, 16, 8, 32)[1:3] == (32, 4)


@pytest.mark.parametrize("args,code", [
    ((4, 24, 4, 256, 12, 100, 2048), _lib.TI_EUNSUPPORTED),   # page neither 1/2/4/8 nor 16k
    ((4, 24, 4, 256, 24, 100, 2048), _lib.TI_EUNSUPPORTED),   # 24: not a multiple of 16
    ((4, 24, 4, 256, 0, 100, 2048), _lib.TI_EUNSUPPORTED),    # no page size
    ((4, 24, 4, 256, 8, 100, 48), _lib.TI_EINVAL),            # split not a multiple of 32
    ((4, 64, 2, 256, 16, 100, 2048), _lib.TI_EUNSUPPORTED),   # group of 32 > 16-row tile
    ((4, 24, 4, 96, 16, 100, 2048), _lib.TI_EUNSUPPORTED),    # head_dim not built
    ((4, 24, 4, 256, 16, 100, 100), _lib.TI_EINVAL),          # split not a multiple of 32
    ((4, 24, 4, 256, 16, 100, 32768), _lib.TI_EINVAL),        # split above the maximum
    ((4, 25, 4, 256, 16, 100, 2048), _lib.TI_EINVAL),         # Hq not a multiple of Hkv
])
def test_decode_plan_rejects(args, code):
    rc = _plan(*args)[0]
    assert rc == code
    assert _lib.load().ti_last_error().decode()


def test_decode_plan_small_pages():
    """Pages of 1, 2, 4 and 8 tokens plan like 16-token pages of the same context: the kernel
    still walks 16-token tiles, so the balanced plan's workgroup count does not change; a split
    is a multiple of 32 tokens whatever the page size."""
    for ps in (1, 2, 4, 8):
        rc, split, wgs, ws = _plan(64, 24, 4, 256, ps, 8192 * 16 // ps // 16, 0)
        assert rc == _lib.TI_OK, ps
        assert (split, wgs) == (0, 256)
        rc, split, ms, _ = _plan(8, 24, 4, 256, ps, 2048 // ps, 512)
        assert (rc, split, ms) == (_lib.TI_OK, 512, 4)


def _decode_abi(variant, batch=0):
    lib = _lib.load()
    return lib.ti_gqa_decode_paged(None, 0, 0, None, None, None, 8, None, None, None, 0, batch,
                                   24, 4, 256, 16, 16, 8, 0, variant, _lib.TI_DTYPE_BF16, None)


def test_decode_cache_policy_flags():
    """The two cache-policy flags: each alone is accepted (an empty batch is then a no-op), both
    together are refused before the plan, as is an unknown flag bit."""
    lib = _lib.load()
    for v in (0, _lib.TI_DECODE_REUSE_KV, _lib.TI_DECODE_STREAM_KV,
              _lib.TI_DECODE_MFMA | _lib.TI_DECODE_STREAM_KV,
              _lib.TI_DECODE_SCALAR | _lib.TI_DECODE_REUSE_KV):
        assert _decode_abi(v) == _lib.TI_OK, hex(v)
    for v in (_lib.TI_DECODE_REUSE_KV | _lib.TI_DECODE_STREAM_KV, 0x40, 3):
        assert _decode_abi(v) == _lib.TI_EINVAL, hex(v)
        assert b"variant" in lib.ti_last_error()
    # A non-empty batch with a valid flag gets as far as the null operands.
    assert _decode_abi(_lib.TI_DECODE_STREAM_KV, batch=2) == _lib.TI_EINVAL
    assert b"null" in lib.ti_last_error()


def test_policy_flag_from_kv_reuse():
    """The Python keyword maps onto the flags: None leaves the choice to the device, True keeps
    K/V cacheable, False streams them."""
    from tileinfer_amd.kernels.gqa_decode_paged import _policy_flag
    assert _policy_flag(None) == 0
    assert _policy_flag(True) == _lib.TI_DECODE_REUSE_KV
    assert _policy_flag(False) == _lib.TI_DECODE_STREAM_KV


def test_append_argument_errors_without_device():
    lib = _lib.load()
    assert lib.ti_kv_append(None, None, 8, 8, None, None, 8, None, 0, 8, 10, 0, None) == _lib.TI_OK
    rc = lib.ti_kv_append(None, None, 8, 8, None, None, 8, None, 4, 8, 10, 7, None)
    assert rc == _lib.TI_EUNSUPPORTED and b"dtype" in lib.ti_last_error()
    rc = lib.ti_kv_append(None, None, 8, 8, None, None, 8, None, 4, 8, 10, 0, None)
    assert rc == _lib.TI_EINVAL and b"null" in lib.ti_last_error()
    with pytest.raises(_lib.TileInferError):
        _lib.check(rc)


def test_python_wrappers_validate_before_launch():
    k = torch.zeros(2, 4, 256, dtype=torch.bfloat16)
    cache = torch.zeros(64, 1024, dtype=torch.bfloat16)
    with pytest.raises(TypeError):
        store_kvcache(k, k, cache, cache, torch.zeros(2, dtype=torch.int64))
    with pytest.raises(ValueError):
        store_kvcache(k, k, cache[:, :512], cache[:, :512], torch.zeros(2, dtype=torch.int32))
    with pytest.raises(ValueError, match="GPU"):
        store_kvcache(k, k, cache, cache, torch.zeros(2, dtype=torch.int32))
    q = torch.zeros(2, 24, 256, dtype=torch.bfloat16)
    kc = torch.zeros(4, 16, 4, 256, dtype=torch.bfloat16)
    bt = torch.zeros(2, 4, dtype=torch.int32)
    sl = torch.ones(2, dtype=torch.int32)
    with pytest.raises(TypeError):
        gqa_decode_paged_fn(q, kc.float(), kc, bt, sl)
    with pytest.raises(ValueError):
        gqa_decode_paged_fn(q, kc, kc, bt, sl, page_size=24)
    with pytest.raises(ValueError, match="GPU"):
        gqa_decode_paged_fn(q, kc, kc, bt, sl)
    cu = torch.tensor([0, 1, 2], dtype=torch.int32)
    with pytest.raises(TypeError):
        gqa_prefill_paged_fn(q, kc, kc, bt, cu.long(), sl)
    with pytest.raises(ValueError):
        gqa_prefill_paged_fn(q, kc, kc, bt, cu[:2], sl)
    with pytest.raises(ValueError):
        gqa_prefill_paged_fn(q, kc, kc, bt, cu, sl, 1, page_size=24)
    with pytest.raises(ValueError, match="GPU"):
        gqa_prefill_paged_fn(q, kc, kc, bt, cu, sl, 1)


def test_qknorm_rope_append_rejects_bad_q_out():
    """A caller-supplied q_out of the wrong shape or dtype is refused before anything runs (the
    kernel would otherwise write q rows past its end)."""
    from tileinfer_amd.kernels.qknorm_rope import qknorm_rope_append
    q = torch.zeros(3, 24, 256, dtype=torch.bfloat16)
    k = torch.zeros(3, 4, 256, dtype=torch.bfloat16)
    w = torch.zeros(256, dtype=torch.bfloat16)
    cs = torch.zeros(64, dtype=torch.bfloat16)
    cache = torch.zeros(64, 1024, dtype=torch.bfloat16)
    slots = torch.zeros(3, dtype=torch.int32)
    for bad in (torch.zeros(2, 24, 256, dtype=torch.bfloat16),   # too few rows
                torch.zeros(3, 24, 256, dtype=torch.float16),    # wrong dtype
                torch.zeros(3, 24, 512, dtype=torch.bfloat16)[:, :, ::2]):  # strided rows
        with pytest.raises(ValueError, match="q_out"):
            qknorm_rope_append(q, k, k, w, w, cs, cs, cache, cache, slots, q_out=bad)


def _prefill_abi(batch=1, total_q=4, max_q=4, hq=24, hkv=4, d=256, ps=16, dtype=0, ptr=None):
    lib = _lib.load()
    return lib.ti_gqa_prefill_paged(ptr, 24 * d, d, ptr, ptr, ptr, 8, ptr, ptr, ptr, 24 * d, d,
                                    None, 0, batch, total_q, max_q, hq, hkv, d, ps, 64, 8, 1,
                                    dtype, None)


def test_prefill_argument_errors_without_device():
    assert _prefill_abi(batch=0) == _lib.TI_OK
    assert _prefill_abi(total_q=0) == _lib.TI_OK
    assert _prefill_abi(dtype=7) == _lib.TI_EUNSUPPORTED
    assert _prefill_abi(d=96) == _lib.TI_EUNSUPPORTED
    for ps in (1, 2, 12, 24):                       # 4, 8 and multiples of 16 are built
        assert _prefill_abi(ps=ps) == _lib.TI_EUNSUPPORTED, ps
    for ps in (4, 8, 32):                           # accepted: fails later, on the null operands
        assert _prefill_abi(ps=ps) == _lib.TI_EINVAL, ps
    assert _prefill_abi(hq=25) == _lib.TI_EINVAL
    # A page must fit 4 GiB (its byte offsets are 32-bit): 256 tokens x 32,768 KV heads x 256
    # bf16 is exactly 4 GiB and refused; half the heads is accepted (then fails on null operands).
    assert _prefill_abi(hq=32768, hkv=32768, ps=256) == _lib.TI_EUNSUPPORTED
    assert b"4 GiB" in _lib.load().ti_last_error()
    assert _prefill_abi(hq=16384, hkv=16384, ps=256) == _lib.TI_EINVAL
    rc = _prefill_abi()
    assert rc == _lib.TI_EINVAL and b"null" in _lib.load().ti_last_error()


def test_gated_prefill_argument_errors_without_device():
    """The gated entry point: a null gate, or gate rows off 16-byte alignment, are rejected before
    anything is launched (fake but aligned device addresses stand in for the tensors)."""
    lib = _lib.load()
    fake = 1 << 20

    def call(gate, gate_st=24 * 256, gate_sh=256):
        return lib.ti_gqa_prefill_paged_gated(fake, 24 * 256, 256, fake, fake, fake, 8, fake, fake,
                                              fake, 24 * 256, 256, None, 0, 1, 4, 4, 24, 4, 256,
                                              16, 64, 8, 1, 0, gate, gate_st, gate_sh, None)
    assert call(None) == _lib.TI_EINVAL and b"null gate" in lib.ti_last_error()
    assert call(fake + 8) == _lib.TI_EINVAL and b"gate" in lib.ti_last_error()
    assert call(fake, gate_sh=4) == _lib.TI_EINVAL and b"gate" in lib.ti_last_error()


def test_prefill_workspace_sizes():
    """The balanced schedule's workspace: plan tables plus two partial slots of 192 rows (head_dim
    256, 12-wave workgroups; 256 rows at 128) per resident workgroup; none past the schedule's
    sequence limit."""
    lib = _lib.load()
    out = ctypes.c_int64(-1)

    def ws(batch, total_q, d=256, hq=24, hkv=4):
        assert lib.ti_gqa_prefill_workspace_bytes(batch, total_q, hq, hkv, d, 16, 512,
                                                  ctypes.byref(out)) == _lib.TI_OK
        return out.value
    one = ws(1, 2048)
    assert one > 256 * 2 * 192 * 256 * 4            # at least one round of partial slots
    assert ws(2, 2048) >= one                       # more pairs, more table rows
    assert ws(8193, 9000) == 0                      # beyond the schedule: run without one
    assert ws(1, 0) == 0
    assert ws(4, 512, d=128, hq=16, hkv=2) > 0
    assert lib.ti_gqa_prefill_workspace_bytes(1, 1, 24, 4, 96, 16, 8, ctypes.byref(out)) == \
        _lib.TI_EUNSUPPORTED


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(RuntimeError, match="no non-HIP fallback"):
        _lib.load(tmp_path / "absent.so")


def test_noalloc_decode_rejects_plans_beyond_its_scratch():
    """A call whose split-K plan needs more than the static scratch is refused with a clear
    error before anything is looked up or launched (no device needed)."""
    lib = _lib.load()
    cap = lib.ti_gqa_decode_scratch_bytes()
    assert cap == 32 << 20
    # 128 query heads over 8 KV heads at 64 x 32k: 256 balanced runs (two whole rounds of 128)
    # x 2 slots x 128 heads x (256 + 2) fp32 = 67.6 MB > 32 MiB, plus the 65 first-tile entries
    # (256-byte rounded).
    s, m, w = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int64()
    _lib.check(lib.ti_gqa_decode_plan(64, 128, 8, 256, 16, 2048, 0, ctypes.byref(s),
                                      ctypes.byref(m), ctypes.byref(w)))
    assert w.value == m.value * 2 * 128 * 258 * 4 + 512 > cap
    rc = lib.ti_gqa_decode_paged_noalloc(None, 0, 0, None, None, None, 2048, None, None, 64, 128,
                                         8, 256, 16, 131072, 2048, 0, 0, 0, None)
    assert rc == _lib.TI_EINVAL
    assert b"no-allocation" in lib.ti_last_error() and b"scratch" in lib.ti_last_error()
    # An empty batch that fits is a no-op.
    assert lib.ti_gqa_decode_paged_noalloc(None, 0, 0, None, None, None, 0, None, None, 0, 24,
                                           4, 256, 16, 0, 0, 0, 0, 0, None) == _lib.TI_OK
    # The same heads with a 128-token bound (16 sequences, 8-page table) take one workgroup per
    # (KV head, sequence) and no scratch, so the size check passes even though the balanced plan
    # of this shape would not fit; the call then fails later for want of a device or pointers.
    _lib.check(lib.ti_gqa_decode_plan(16, 128, 8, 256, 16, 8, 0, ctypes.byref(s),
                                      ctypes.byref(m), ctypes.byref(w)))
    assert (s.value, m.value) == (0, 0) and w.value > cap
    rc = lib.ti_gqa_decode_paged_noalloc(None, 0, 0, None, None, None, 8, None, None, 16, 128,
                                         8, 256, 16, 1024, 8, 0, 0, 0, None)
    assert rc != _lib.TI_OK and b"scratch" not in lib.ti_last_error()


def test_decode_plan_per_pair_round_rule_without_device():
    """Bounds of at most 512 tokens take one workgroup per (KV head, sequence) when those pairs
    fill three quarters to all of one round (no device here: the library assumes 256 CUs), and
    the balanced plan just outside either edge."""
    assert _plan(64, 24, 4, 256, 16, 32, 0)[:3] == (0, 0, 0)     # 256 pairs, a 512-token bound
    assert _plan(48, 24, 4, 256, 16, 32, 0)[:3] == (0, 0, 0)     # 192 pairs: three quarters
    assert _plan(32, 32, 8, 128, 8, 50, 0)[:3] == (0, 0, 0)      # pages of 8, a 400-token bound
    assert _plan(47, 24, 4, 256, 16, 32, 0)[:3] == (0, 0, 256)   # 188 pairs: balanced
    assert _plan(65, 24, 4, 256, 16, 32, 0)[:3] == (0, 0, 256)   # 260 pairs: over one round
    assert _plan(64, 24, 4, 256, 16, 33, 0)[:3] == (0, 0, 256)   # a 528-token bound


def test_fused_append_decode_argument_errors_without_device():
    """ti_gqa_decode_paged_append refuses bad append operands on the host, before anything is
    launched (stand-in device addresses, never dereferenced: every call below fails first)."""
    lib = _lib.load()
    s, m, w = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int64()
    _lib.check(lib.ti_gqa_decode_plan(2, 24, 4, 256, 16, 8, 0, ctypes.byref(s), ctypes.byref(m),
                                      ctypes.byref(w)))
    fake = 1 << 20  # 16-byte aligned stand-in address
    nb, rows = 16, 16 * 16

    def call(key=fake, stride=1024, slots=fake, num_slots=rows, variant=0):
        return lib.ti_gqa_decode_paged_append(
            fake, 24 * 256, 256, fake, fake, fake, 8, fake, fake, fake, w.value, 2, 24, 4, 256,
            16, nb, 8, 0, variant, 0, key, fake, stride, 1024, slots, num_slots, None)

    assert call(slots=None) == _lib.TI_EINVAL and b"slot_mapping" in lib.ti_last_error()
    assert call(num_slots=rows + 1) == _lib.TI_EINVAL and b"num_slots" in lib.ti_last_error()
    assert call(key=fake + 8) == _lib.TI_EINVAL and b"aligned" in lib.ti_last_error()
    assert call(stride=1000) == _lib.TI_EINVAL
    assert call(variant=_lib.TI_DECODE_SCALAR) == _lib.TI_EUNSUPPORTED
