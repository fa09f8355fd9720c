"""Write the committed golden fixtures (run from the repository root):

    python tests/golden/make_fixtures.py

chunk_gla_config1.npz: BASELINE config 1 -- chunk_gla forward, fp32, B=2, T=512, H=4,
K=V=64, chunk 64; q, k, v ~ N(0,1) from NumPy PCG64(1001) with q multiplied by K^-1/2
after drawing; scale=None, so the default K^-1/2 applies on top (the config's wording is
ambiguous; this is the recorded choice); g = logsigmoid(N(0,1)) / 16; no h0;
output_final_state=True.  Outputs o [2,512,4,64] and ht [2,4,64,64] of the float64
oracle (a restatement of tops/cpu/ops/gla/chunk.py), stored as float32.

The reference's own implementation cannot run here (it needs jax), so the values come from
the oracle, which the CPU tests pin against the naive recurrence and torch autograd.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (ROOT, os.path.dirname(HERE)):
    if p not in sys.path:
        sys.path.insert(0, p)

CONFIG1 = dict(B=2, T=512, H=4, K=64, V=64, seed=1001)


def config1_inputs():
    from _inputs import logsigmoid
    B, T, H, K, V, seed = (CONFIG1[x] for x in ("B", "T", "H", "K", "V", "seed"))
    rng = np.random.Generator(np.random.PCG64(seed))
    q = (rng.standard_normal((B, T, H, K)) * K ** -0.5).astype(np.float32)
    k = rng.standard_normal((B, T, H, K)).astype(np.float32)
    v = rng.standard_normal((B, T, H, V)).astype(np.float32)
    g = (logsigmoid(rng.standard_normal((B, T, H, K))) / 16).astype(np.float32)
    return dict(q=q, k=k, v=v, g=g)


def config1_oracle():
    from oracle import gla as O
    d = config1_inputs()
    o, ht = O.chunk_gla(d["q"], d["k"], d["v"], d["g"], scale=None, initial_state=None,
                        output_final_state=True, chunk_size=64)
    return o, ht


def main():
    o, ht = config1_oracle()
    path = os.path.join(HERE, "chunk_gla_config1.npz")
    np.savez_compressed(path, o=o.astype(np.float32), ht=ht.astype(np.float32),
                        seed=np.int64(CONFIG1["seed"]))
    print(f"wrote {path}")


if __name__ == "__main__":
    main()
