"""``AdaptQAttention``: the reference's PyTorch module (adaptq/torch_adapter.py:20-113)
over the GPU KV cache.

Same constructor, ``forward(q, k, v)`` on (1, heads, dim) tensors and
``reset_cache()``.  The reference moves every tensor to the CPU and back
(torch_adapter.py:100-108); here tensors on a ROCm device stay there: the
step appends k, v and decodes q through the whole-MHA device entry points on
torch's current stream, so no host copy is made.  CPU tensors take the
Engine's host path.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from .core import Engine


class AdaptQAttention(nn.Module):
    def __init__(self, dim: int, heads: int, k_bits: int = 4, v_bits: int = 4,
                 capacity: int = 4096, seed: int = 42):
        super().__init__()
        self.dim = dim
        self.heads = heads
        self.k_bits = k_bits
        self.v_bits = v_bits
        self.engine = Engine(dim=dim, heads=heads, k_bits=k_bits, v_bits=v_bits,
                             capacity=capacity, seed=seed)

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        """q, k, v: (1, heads, dim).  Appends k, v, then returns the attention
        output for q, (1, heads, dim), on q's device and dtype."""
        if q.dim() != 3 or k.dim() != 3 or v.dim() != 3:
            raise ValueError(
                "AdaptQAttention.forward() expects 3D tensors (batch, heads, dim). "
                f"Got shapes q={tuple(q.shape)}, k={tuple(k.shape)}, v={tuple(v.shape)}.")
        if q.size(0) != 1:
            raise ValueError(
                f"AdaptQAttention does not support batch_size > 1 (got {q.size(0)}). "
                "Create one AdaptQAttention per sequence.")
        if q.size(1) != self.heads or q.size(2) != self.dim:
            raise ValueError(f"Expected q shape (1, {self.heads}, {self.dim}), "
                             f"got {tuple(q.shape)}.")
        if k.shape != q.shape:
            raise ValueError(f"Expected k shape {tuple(q.shape)}, got {tuple(k.shape)}.")
        if v.shape != q.shape:
            raise ValueError(f"Expected v shape {tuple(q.shape)}, got {tuple(v.shape)}.")

        if q.is_cuda:
            kd = k.detach()[0].to(torch.float32).contiguous()
            vd = v.detach()[0].to(torch.float32).contiguous()
            qd = q.detach()[0].to(torch.float32).contiguous()
            out = torch.empty_like(qd)
            stream = torch.cuda.current_stream(q.device).cuda_stream
            ctx = self.engine._ctx
            ctx.append_all_device(kd.data_ptr(), vd.data_ptr(), 1, self.engine.pos, stream)
            self.engine.pos += 1
            ctx.compute_all_device(qd.data_ptr(), out.data_ptr(), stream)
            return out.unsqueeze(0).to(dtype=q.dtype)

        k_np = k.detach().float().cpu().numpy()[0]
        v_np = v.detach().float().cpu().numpy()[0]
        q_np = q.detach().float().cpu().numpy()[0]
        self.engine.append(k_np, v_np)
        out_np = self.engine.compute(q_np)
        return torch.from_numpy(out_np).unsqueeze(0).to(device=q.device, dtype=q.dtype)

    def reset_cache(self) -> None:
        """Clear the KV cache; call between independent sequences."""
        self.engine.reset()
