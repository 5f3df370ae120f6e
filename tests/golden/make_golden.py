"""Writes the config-1 golden fixtures: input hashes and the oracle's decode output.

Run from the repository root: ``python tests/golden/make_golden.py``. Inputs are regenerated from
seeds by tileinfer_amd.workloads.config1 (torch CPU generator); the SHA-256 of every input tensor
is recorded so that generator drift fails loudly instead of silently changing the expected values.
The expected output is the oracle's restatement of the reference recipe (oracle/ref_torch.py:
append, then decode), stored as the raw bf16 bits.
"""
import hashlib
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle.ref_torch import ref_gqa_decode_paged, ref_store_kvcache  # noqa: E402
from tileinfer_amd.workloads import config1  # noqa: E402


def sha(t) -> str:
    return hashlib.sha256(t.contiguous().view(-1).view(dtype=__import__("torch").uint8).numpy()
                          .tobytes()).hexdigest()


def input_hashes(step) -> dict:
    return {name: sha(getattr(step, name)) for name in
            ("q", "k_new", "v_new", "slot_mapping", "block_table", "seqlen", "k_cache", "v_cache")}


def expected(step):
    kc, vc = step.k_cache.clone(), step.v_cache.clone()
    ref_store_kvcache(step.k_new, step.v_new, kc.view(-1, 1024), vc.view(-1, 1024),
                      step.slot_mapping)
    return ref_gqa_decode_paged(step.q, kc, vc, step.block_table, step.seqlen, 16)


def main():
    for ctx in (512, 513):
        step = config1(ctx=ctx)
        out = expected(step)
        bits = out.view(-1).view(dtype=__import__("torch").int16).numpy().astype(np.uint16)
        np.save(HERE / f"config1_ctx{ctx}_out.npy", bits.reshape(24, 256))
        meta = {"config": 1, "seed": step.meta["seed"], "ctx": ctx,
                "slot": int(step.slot_mapping[0]), "inputs_sha256": input_hashes(step),
                "output_sha256": sha(out), "output_shape": [1, 24, 256], "dtype": "bfloat16"}
        (HERE / f"config1_ctx{ctx}.json").write_text(json.dumps(meta, indent=1) + "\n")
        print(f"ctx {ctx}: slot {meta['slot']}, out sha {meta['output_sha256'][:16]}")


if __name__ == "__main__":
    main()
