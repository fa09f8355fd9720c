"""BASELINE config 1 against the committed golden fixture (tests/golden/chunk_gla_config1.npz).

CPU: the float64 oracle regenerates the fixture from the seeded inputs (guards the oracle
and the input generator against drift).  GPU: the HIP chunk_gla forward in fp32 matches the
fixture within the fp32 tolerance (rel L2 <= 1e-4).
"""
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_fixtures as MF  # noqa: E402
from _closed_forms import rel  # noqa: E402

FIX = os.path.join(HERE, "golden", "chunk_gla_config1.npz")


def _fixture():
    with np.load(FIX, allow_pickle=False) as z:
        return z["o"].astype(np.float64), z["ht"].astype(np.float64), int(z["seed"])


def test_oracle_regenerates_config1_fixture():
    o_ref, ht_ref, seed = _fixture()
    assert seed == MF.CONFIG1["seed"]
    assert o_ref.shape == (2, 512, 4, 64) and ht_ref.shape == (2, 4, 64, 64)
    o, ht = MF.config1_oracle()
    assert rel(o, o_ref) < 1e-6 and rel(ht, ht_ref) < 1e-6


@pytest.mark.gpu
def test_hip_chunk_gla_config1_matches_fixture(cuda_device):
    import torch
    from tops.ops.gla import chunk_gla
    d = MF.config1_inputs()
    q, k, v, g = (torch.from_numpy(d[x]).to(cuda_device) for x in ("q", "k", "v", "g"))
    o, ht = chunk_gla(q, k, v, g, output_final_state=True, chunk_size=64)
    torch.cuda.synchronize()
    o_ref, ht_ref, _ = _fixture()
    eo = rel(o.double().cpu().numpy(), o_ref)
    eh = rel(ht.double().cpu().numpy(), ht_ref)
    print(f"config 1: o rel {eo:.2e}, ht rel {eh:.2e}")
    assert eo <= 1e-4 and eh <= 1e-4
