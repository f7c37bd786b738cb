"""scatter_kv on the GPU vs the oracle (bit-exact copy)."""
import numpy as np
import pytest
import torch

import mugen_amd
from oracle import oracle as O
from tests import cases as C

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("count,offset", [(576, 576 * 37), (1024, 0), (131, 5), (7, 999), (8 * 4 * 128, 8 * 4 * 128 * 3)])
def test_scatter_kv_bit_exact(device, count, offset):
    C.say(f"scatter_kv count={count} offset={offset}")
    rng = np.random.default_rng(count)
    src = rng.integers(0, 65535, count, dtype=np.uint16)
    dst = rng.integers(0, 65535, 40000, dtype=np.uint16)
    ref = O.scatter_kv(src, dst, offset, count)
    s = C.to_dev(src, C.F16, device)
    d = C.to_dev(dst, C.F16, device)
    mugen_amd.scatter_kv(s, d, offset)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(d.cpu().view(torch.int16).numpy().view(np.uint16), ref)
