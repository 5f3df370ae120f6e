"""Pins the restated reference decode-metadata builder (CPU only) against kv_layout's builders,
whose slot formula and padding are checked against the definition in tests/test_engine.py."""
import pytest
import torch

from oracle.ref_metadata import RefDecodePrep
from tileinfer_amd.engine import PagedKVManager, Sequence
from tileinfer_amd.engine import kv_layout as kl


@pytest.mark.parametrize("bsz", [5, 8])
def test_ref_prepare_decode_equals_host_builder(bsz):
    m = PagedKVManager(500, 16)
    seqs = [Sequence(list(range(n))) for n in (1, 16, 17, 300, 1000)]
    for s in seqs:
        assert m.admit(s)
        m.finish_chunk(s, s.num_tokens)
        s.append_token(5)
        m.append_slot(s)
    ref = RefDecodePrep(8, 80)
    rs, rt, rc = ref(seqs, 16, bsz=bsz)
    hs, ht, hc = kl.decode_metadata(seqs, 16, device="cpu", pad_to=bsz, width=80)
    assert torch.equal(rs, hs) and torch.equal(rt, ht) and torch.equal(rc, hc)
    # The slot is the definition's: block_table[pos // 16] * 16 + pos % 16, pos = num_tokens - 1.
    for i, s in enumerate(seqs):
        pos = s.num_tokens - 1
        assert int(rs[i]) == s.block_table[pos // 16] * 16 + pos % 16
