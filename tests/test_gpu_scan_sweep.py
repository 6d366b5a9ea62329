"""A seeded sweep of small, irregular selective-scan shapes on the GPU against
the oracle: batch 1-3, channel counts that leave the last 64-channel block
part-filled, lengths from 1 to 700 (aligned and not, so both the buffer-range
and the pointer paths run, with and without the sequence split and its
summary parts), 1 to 40 states, bf16 and fp32, with and without z, lengths,
h_init and dh_last.  Each case draws its configuration from its own seed, so
a failure names a reproducible case."""
import random

import pytest
import torch

from tests.test_gpu_scan import run_case

pytestmark = pytest.mark.gpu


def _config(seed):
    g = random.Random(seed)
    batch = g.choice([1, 1, 2, 3])
    dim = g.choice([16, 64, 80, 130, 200])
    seqlen = g.choice([1, 7, 16, 33, 96, 128, 200, 257, 300, 513, 700])
    nstate = g.choice([1, 2, 5, 8, 12, 16, 16, 16, 24, 40])
    dtype = g.choice([torch.float32, torch.bfloat16])
    with_z = g.random() < 0.7
    side = g.choice(["right", "left"])
    length = None
    if g.random() < 0.5:
        length = torch.tensor([g.randint(0, seqlen) for _ in range(batch)], dtype=torch.int64)
    return dict(batch=batch, dim=dim, seqlen=seqlen, nstate=nstate, dtype=dtype, with_z=with_z,
                padding_side=side, length=length, h_init=g.random() < 0.5,
                dlast=g.random() < 0.5)


@pytest.mark.parametrize("seed", range(200))
def test_sweep(cuda, seed):
    c = _config(1000 + seed)
    run_case(cuda, c["batch"], c["dim"], c["seqlen"], c["nstate"], c["dtype"], seed=2000 + seed,
             with_z=c["with_z"], h_init=c["h_init"], length=c["length"],
             padding_side=c["padding_side"], dlast=c["dlast"])
