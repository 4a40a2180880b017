"""Writes tests/golden/smollm_ref_fp32.json from the reference's own emitted C99 SmolLM module.

Run in the build container only (needs /root/reference for oracle/_ref):
    make -C oracle && python tests/golden/make_golden.py

The fixture is data: seeded synthetic fp32 weights (the build's recipe) pushed through
velox_SmolLM_135M_prefill of /root/reference/src/runners/tinystories_smollm.c, compiled in place;
per position it records the argmax, the sha256 of the 49152 fp32 logits, the first 16 logits and
the top-5. tests/test_oracle.py requires the oracle to reproduce it bit for bit.
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import pyoracle as po  # noqa: E402

SEED, SIGMA, NORM_SIGMA, N_POS = 7, 0.02, 0.1, 4


def main():
    ref = po.RefSmolLM(SEED, SIGMA, NORM_SIGMA)
    toks = [int(t) for t in po.prompt_tokens(SEED, N_POS, 49152)]
    steps = []
    for pos, tok in enumerate(toks):
        nxt = ref.step(tok, pos)
        lg = ref.logits.copy()
        top = np.argsort(-lg, kind="stable")[:5]
        steps.append({
            "pos": pos, "token_in": tok, "argmax": nxt,
            "logits_sha256": hashlib.sha256(lg.tobytes()).hexdigest(),
            "logits_head": [float(v) for v in lg[:16]],
            "top5": [[int(i), float(lg[i])] for i in top],
        })
    ref.close()
    out = {
        "source": "velox_SmolLM_135M_prefill, /root/reference/src/runners/tinystories_smollm.c:532 "
                  "(compiled by oracle/Makefile, -O2 -mavx2 -mfma -fopenmp -ffp-contract=off)",
        "model": "SmolLM-135M shapes, fp32 weights N(0, sigma) from the build's counter RNG, norm gains N(1, norm_sigma)",
        "seed": SEED, "sigma": SIGMA, "norm_sigma": NORM_SIGMA, "steps": steps,
    }
    with open(os.path.join(HERE, "smollm_ref_fp32.json"), "w") as f:
        json.dump(out, f, indent=1)
    print("wrote", len(steps), "positions")


if __name__ == "__main__":
    main()
