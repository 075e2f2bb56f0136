"""TurboQuant host-side export vs the oracle (no GPU needed).

pi_tq_generate builds the per-head rotation and QJL matrices of
TurboQuant::new (src/turboquant/mod.rs:76-103) on the host; the device
quantizer is only bit-compatible with the reference if these matrices are
identical to the restatement's, bit for bit.
"""
import numpy as np
import pytest

from oracle import oracle as o
from powerinfer_x64_amd import runtime as rt


@pytest.mark.parametrize("dim,seed", [(128, 0xCAFEBABE), (128, 0xCAFEBABE + 7), (16, 123),
                                      (64, 456), (256, 0xCAFEBABE + 1)])
def test_generate_matches_oracle_bitwise(dim, seed):
    R, G = rt.tq_generate(dim, seed)
    R2, G2 = o.tq_matrices(dim, seed)
    assert np.array_equal(R.view(np.uint32), R2.view(np.uint32))
    assert np.array_equal(G.view(np.uint32), G2.view(np.uint32))


def test_generate_rejects_bad_arguments():
    with pytest.raises(rt.InvalidArg):
        rt.tq_generate(0, 1)
