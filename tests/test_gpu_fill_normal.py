"""GPU: the device input generator (tl_fill_normal_f16) against the oracle's
(orc_fill_normal_f16, splitmix64 -> Box-Muller -> fp16 RNE): the same fp16
bits element for element, for whole streams and for ranges that start and
end on odd elements, and NormalStreams continuing a stream across draws."""
import numpy as np
import pytest
import torch

import workloads
from devutil import empty_dev, stream, to_host

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed,first,n,std", [
    (workloads.seed(3, 1), 0, 1 << 22, 1.0),
    (workloads.seed(2, 2), 12345, 100001, 0.5),
    (workloads.seed(5, 0), 0, 1, 1.0),
    (workloads.seed(5, 0), 7, 2, 1.0),
    (2**64 - 5, 999, 4097, 3.0),
])
def test_device_stream_equals_the_oracle_generator(tl, orc, seed, first, n, std):
    out = empty_dev((n,))
    tl.fill_normal(seed, first, std, out.data_ptr(), n, stream())
    got = to_host(out)
    ref = orc.normal_f16(seed, (first + n,), std)[first:]
    assert np.array_equal(got, ref), int(np.count_nonzero(got != ref))
    if n >= 1 << 20:  # a normal sample: mean ~ 0, std ~ std
        x = got.view(np.float16).astype(np.float64)
        assert abs(x.mean()) < 5e-3 and abs(x.std() - std) < 5e-3 * std


def test_normal_streams_continue_across_draws(tl, orc):
    ns = tl.NormalStreams(stream())
    a = ns.draw(11, (3, 5))
    b = ns.draw(11, (7,), stddev=1.0)
    c = ns.draw(12, (4,))
    ref11 = orc.normal_f16(11, (22,))
    assert np.array_equal(to_host(a).reshape(-1), ref11[:15])
    assert np.array_equal(to_host(b), ref11[15:22])
    assert np.array_equal(to_host(c), orc.normal_f16(12, (4,)))
    assert ns.offset == {11: 22, 12: 4}
    torch.cuda.synchronize()
