"""Writes tests/golden/e2e_2b_seed0.npz: greedy decode of the 2B-shaped model computed by the
oracle (the CPU restatement, not the GPU path).

Workload (the one bench.py measures): Qwen3.5-2B shapes, synthetic weights N(0, 0.02) drawn
with seed 0 and quantised to Q8F, a 512-token uniform random prompt (numpy default_rng(0)), then
512 greedy steps.  Stored: the prompt, the 513 greedy ids (the token after the prompt and the 512
decoded ones) and, per id, the oracle's top-1 minus top-2 logit margin (small margins are where a
rounding difference could legitimately flip a greedy choice).

    python tests/golden/make_e2e_2b.py        # ~10 minutes on 8 cores
"""
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "qwen-3.5_amd"))
sys.path.insert(0, ROOT)

import oracle as O  # noqa: E402
import q35  # noqa: E402

N_PROMPT, N_NEW, SEED = 512, 512, 0


def main():
    d = q35.dims_2b()
    prompt = np.random.default_rng(SEED).integers(0, d.vocab, N_PROMPT).astype(np.int32)
    t0 = time.time()
    ref = O.Model(O.cfg_from_dims(d), lambda name, n: q35.synth_model_tensor(d, SEED, name, n), N_PROMPT + N_NEW + 64)
    print(f"weights built in {time.time() - t0:.0f} s", flush=True)
    t0 = time.time()
    toks, margins = ref.generate(prompt, N_NEW)
    print(f"{N_PROMPT} + {N_NEW} steps in {time.time() - t0:.0f} s; min margin {margins.min():.4g}", flush=True)
    out = os.path.join(HERE, "e2e_2b_seed0.npz")
    np.savez_compressed(out, prompt=prompt, tokens=toks.astype(np.int32), margins=margins.astype(np.float32),
                        seed=np.int64(SEED))
    print("wrote", out)


if __name__ == "__main__":
    main()
