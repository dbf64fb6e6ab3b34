"""Device router: the routing half of ``routes_and_shared``
(kaggle/qwen38_tpu/math.py:277-281) on the GPU, feeding ``expert_parallel``.

``routes(logits, top_k, active=None)`` takes the FP32 router logits [B, E]
(the reference computes them with ``linear`` in FP32) and returns ids int32
[B, k] and BF16 weights [B, k]: softmax, top_k (lower id first on ties),
weights divided by their sum, inactive rows zeroed, RNE to BF16.
"""

import torch

from . import _lib


def routes(logits, top_k, active=None):
    if not isinstance(logits, torch.Tensor) or logits.device.type != "cuda" or logits.ndim != 2:
        raise ValueError("logits must be a GPU tensor [tokens, experts]")
    logits = logits.to(torch.float32).contiguous()
    B, E = logits.shape
    if type(top_k) is not int or not 1 <= top_k <= min(E, 32) or E > 1024:
        raise ValueError("need 1 <= top_k <= min(experts, 32) and experts <= 1024")
    act = None
    if active is not None:
        act = active.to(device=logits.device, dtype=torch.uint8).contiguous()
        if act.shape != (B,):
            raise ValueError("active must hold one flag per token")
    ids = torch.empty((B, top_k), dtype=torch.int32, device=logits.device)
    weights = torch.empty((B, top_k), dtype=torch.bfloat16, device=logits.device)
    lib = _lib.load()
    with torch.cuda.device(logits.device):
        rc = lib.q6moe_route_topk(logits.data_ptr(), B, E, top_k, None if act is None else act.data_ptr(),
                                  ids.data_ptr(), weights.data_ptr(), _lib.stream_handle(logits.device))
    _lib.check(rc, "route_topk")
    return ids, weights
