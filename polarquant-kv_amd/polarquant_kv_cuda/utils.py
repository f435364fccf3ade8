"""src/polarquant_kv_cuda/utils.py:6-10."""

import torch


def cosine_similarity_gpu(a: torch.Tensor, b: torch.Tensor) -> float:
    return torch.nn.functional.cosine_similarity(a.flatten().float(), b.flatten().float(), dim=0).item()
