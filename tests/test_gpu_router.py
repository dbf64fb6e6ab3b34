"""GPU parity of the device router against the routing oracle.

The softmax sum runs in a different order from the oracle's, so a probability
can differ by one FP32 ulp: ids must match exactly (the logits here have no
near-ties), weights to one BF16 ulp with almost all of them bit-identical.
"""

import numpy as np
import pytest
import torch

from oracle import routing as oracle_routing
from q6moe.router import routes

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("tokens,experts,top_k", [(8, 128, 8), (300, 64, 6), (5, 256, 32), (3, 7, 7), (1, 1, 1),
                                                   # the reference model's router (config.py:17-18) and the
                                                   # widest layer the kernels take
                                                   (64, 512, 10), (2048, 512, 10), (9, 257, 3), (17, 1024, 32)])
def test_router_matches_oracle(device, tokens, experts, top_k):
    rng = np.random.default_rng(tokens * experts + top_k)
    logits = rng.standard_normal((tokens, experts)).astype(np.float32)
    active = rng.random(tokens) > 0.2
    active[0] = True
    ids, w = routes(torch.from_numpy(logits).to(device), top_k, torch.from_numpy(active).to(device))
    want_ids, want_w = oracle_routing.route(logits, top_k, active)
    np.testing.assert_array_equal(ids.cpu().numpy(), want_ids)
    got = w.float().cpu().numpy()
    np.testing.assert_allclose(got, want_w, rtol=2 ** -7, atol=0)
    assert np.mean(got == want_w) >= 0.98


def test_router_ties_pick_the_lower_id(device):
    logits = np.zeros((2, 16), np.float32)
    logits[0, [3, 9, 12]] = 2.0      # three-way tie at the top
    logits[1, :] = 1.0               # all equal
    ids, _ = routes(torch.from_numpy(logits).to(device), 4)
    want_ids, _ = oracle_routing.route(logits, 4)
    np.testing.assert_array_equal(ids.cpu().numpy(), want_ids)


def test_router_rejects_more_than_1024_experts(device):
    with pytest.raises(ValueError, match="experts <= 1024"):
        routes(torch.zeros((2, 1025), device=device), 4)
