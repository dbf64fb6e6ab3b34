"""The streaming expert loader builds the same unit-major tables as pack_experts."""

import numpy as np
import pytest
import torch

from q6moe.experts import pack_experts
from q6moe.loader import stream_expert_table
from q6moe.synth import moe_layer

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("qtype,down_qtype,group", [("Q6_K", "Q6_K", 3), ("Q4_K", "Q8_0", 8), ("Q6_K", "Q8_0", 1)])
def test_streamed_tables_equal_packed_tables(device, qtype, down_qtype, group):
    L = moe_layer(seed=5, experts=7, top_k=2, hidden=512, intermediate=256, tokens=1, qtype=qtype,
                  down_qtype=down_qtype, pack=False)
    for name, q, rows, width in (("gate", qtype, 256, 512), ("down", down_qtype, 512, 256)):
        raw = np.ascontiguousarray(L[name]).reshape(-1)
        reads = []

        def read(offset, size):
            reads.append((offset, size))
            return raw[offset:offset + size].tobytes()

        got = stream_expert_table(read, q, 7, rows, width, device, group_experts=group)
        want = pack_experts(L[name], q, rows, width, device)
        torch.testing.assert_close(got.data, want.data, rtol=0, atol=0)
        assert sum(s for _, s in reads) == raw.size and max(s for _, s in reads) <= group * raw.size // 7
