"""Quantized LLaMA block decode over libsgq.so (ctypes).

Mirrors the reference's LLaMABlock (include/sovereigngrad/models.hpp:197-224)
with every nn::Linear replaced by QuantizedLinear4Bit (nn.hpp:965-1001): the
same seven projections (attention q, k, v, out; SwiGLU gate, up, down), the
two RMSNorm weights and CausalSelfAttention's scale
1 / sqrt((float)(embed_dim / num_heads)) (nn.hpp:518).  The reference has no
KV cache -- NanoLLaMA::generate reruns the whole sequence every token
(models.hpp:270-302) -- so decode() takes one new token per sequence and a
key/value cache, and returns what the reference's forward gives for that
token's row.
"""
from __future__ import annotations

import ctypes
from typing import Dict, Optional, Sequence

import torch

from . import (QuantizedTensor, _check, _dev_f32, _linear_ws, _ptr, _stream, load_library, pack_int4,
               quantize_int4)

PROJECTIONS = ("q", "k", "v", "out", "gate", "up", "down")


class Int4Linear(ctypes.Structure):
    """sgq_int4_linear (include/sgq.h)."""
    _fields_ = [("packed", ctypes.c_void_p), ("devscales", ctypes.c_void_p), ("bias", ctypes.c_void_p)]


class LlamaBlockInt4(ctypes.Structure):
    """sgq_llama_block_int4 (include/sgq.h)."""
    _fields_ = [("D", ctypes.c_int64), ("H", ctypes.c_int64), ("group_size", ctypes.c_int64),
                ("eps", ctypes.c_float), ("attn_scale", ctypes.c_float),
                ("norm1", ctypes.c_void_p), ("norm2", ctypes.c_void_p),
                ("q", Int4Linear), ("k", Int4Linear), ("v", Int4Linear), ("o", Int4Linear),
                ("gate", Int4Linear), ("up", Int4Linear), ("down", Int4Linear)]


def projection_shapes(D: int, H: int):
    """[in, out] of each projection in PROJECTIONS order."""
    return {"q": (D, D), "k": (D, D), "v": (D, D), "out": (D, D), "gate": (D, H), "up": (D, H), "down": (H, D)}


def attention_scale(embed_dim: int, num_heads: int) -> float:
    """CausalSelfAttention::scale: 1.0f / std::sqrt((float)(embed_dim / num_heads)) (nn.hpp:518)."""
    import numpy as np

    return float(np.float32(1.0) / np.sqrt(np.float32(embed_dim // num_heads)))


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-5, out: Optional[torch.Tensor] = None):
    """rms_norm (src/ops.cpp:1532-1556) over the last dimension, on the device."""
    lib = load_library()
    x = _dev_f32(x)
    if x.dim() < 2:
        raise ValueError("RMSNorm requires at least 2D tensor!")  # src/ops.cpp:1533
    D = x.shape[-1]
    y = out if out is not None else torch.empty_like(x)
    _check(lib.sgq_rms_norm(_ptr(x), x.numel() // D, D, _ptr(_dev_f32(weight)), ctypes.c_float(eps), _ptr(y),
                            _stream(x.device)))
    return y


class KVCache:
    """Per-block key/value cache: [B, max_tokens, D] fp32 each, plus the
    per-sequence positions (int32, device) that decode() reads."""

    def __init__(self, B: int, max_tokens: int, D: int, device, layers: int = 1):
        self.B, self.max_tokens, self.D = B, max_tokens, D
        self.k = [torch.empty((B, max_tokens, D), dtype=torch.float32, device=device) for _ in range(layers)]
        self.v = [torch.empty((B, max_tokens, D), dtype=torch.float32, device=device) for _ in range(layers)]
        self.pos = torch.zeros(B, dtype=torch.int32, device=device)


class QuantizedLLaMABlock:
    """LLaMABlock with INT4-grouped projections, decoded one token at a time."""

    def __init__(self, D: int, H: int, num_heads: int, group_size: int, weights: Dict[str, QuantizedTensor],
                 biases: Dict[str, Optional[torch.Tensor]], norm1: torch.Tensor, norm2: torch.Tensor,
                 eps: float = 1e-5):
        shapes = projection_shapes(D, H)
        for name in PROJECTIONS:
            w = weights[name]
            if (w.rows, w.cols) != shapes[name] or w.bits != 4 or w.group_size != group_size:
                raise ValueError(f"projection {name}: expected INT4 g{group_size} {shapes[name]}")
            if w.devscales is None:
                raise ValueError(f"projection {name}: the block needs the tiled INT4 layout")
        self.D, self.H, self.group_size, self.eps = D, H, group_size, eps
        self.num_heads = num_heads
        self.weights = weights
        self.biases = {k: (None if v is None else _dev_f32(v).reshape(-1).contiguous()) for k, v in biases.items()}
        self.norm1, self.norm2 = _dev_f32(norm1).reshape(-1), _dev_f32(norm2).reshape(-1)
        self.attn_scale = attention_scale(D, num_heads)
        st = LlamaBlockInt4()
        st.D, st.H, st.group_size = D, H, group_size
        st.eps, st.attn_scale = eps, self.attn_scale
        st.norm1, st.norm2 = _ptr(self.norm1), _ptr(self.norm2)
        for name, field in zip(PROJECTIONS, ("q", "k", "v", "o", "gate", "up", "down")):
            w = weights[name]
            setattr(st, field, Int4Linear(_ptr(w.packed), _ptr(w.devscales), _ptr(self.biases.get(name))))
        self._struct = st

    @classmethod
    def from_float(cls, W: Dict[str, torch.Tensor], b: Dict[str, Optional[torch.Tensor]], norm1, norm2,
                   num_heads: int, group_size: int = 32, eps: float = 1e-5) -> "QuantizedLLaMABlock":
        """Quantizes each projection's [in, out] weight on the device, as
        QuantizedLinear4Bit::from_float does (nn.hpp:984-992)."""
        D, H = W["gate"].shape
        q = {k: quantize_int4(W[k], group_size, keep_qdata=False) for k in PROJECTIONS}
        return cls(D, H, num_heads, group_size, q, b, norm1, norm2, eps)

    @classmethod
    def from_codes(cls, codes: Dict[str, torch.Tensor], scales: Dict[str, torch.Tensor],
                   b: Dict[str, Optional[torch.Tensor]], norm1, norm2, num_heads: int, group_size: int,
                   eps: float = 1e-5) -> "QuantizedLLaMABlock":
        """From reference-layout fp32 codes and scales (a state_dict's qdata / scales)."""
        D, H = codes["gate"].shape
        q = {k: pack_int4(codes[k], scales[k], group_size) for k in PROJECTIONS}
        return cls(D, H, num_heads, group_size, q, b, norm1, norm2, eps)

    def workspace_bytes(self, B: int, max_len: int) -> int:
        return int(load_library().sgq_llama_decode_workspace_bytes(B, self.D, self.H, max_len))

    def decode(self, x: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, pos: torch.Tensor,
               max_len: int, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """x [B, D]: one new token per sequence; pos [B] int32 (tokens already
        cached).  Writes the new keys/values at pos and returns the block output
        [B, D].  The caller advances pos after all layers of the step."""
        lib = load_library()
        x = _dev_f32(x)
        B = x.shape[0]
        if x.shape[1] != self.D:
            raise ValueError("x must be [B, D]")
        if k_cache.dtype != torch.float32 or v_cache.dtype != torch.float32 or k_cache.shape != v_cache.shape:
            raise ValueError("caches must be fp32 [B, max_tokens, D]")
        if k_cache.shape[0] != B or k_cache.shape[2] != self.D or not k_cache.is_contiguous():
            raise ValueError("caches must be contiguous [B, max_tokens, D]")
        if pos.dtype != torch.int32 or pos.numel() != B or not pos.is_cuda:
            raise ValueError("pos must be a device int32 tensor of B positions")
        y = out if out is not None else torch.empty_like(x)
        dev = x.device
        ws, nws = _linear_ws.get(self.workspace_bytes(B, max_len), dev)
        _check(lib.sgq_llama_block_decode_int4(ctypes.byref(self._struct), _ptr(x), _ptr(y), B, _ptr(k_cache),
                                               _ptr(v_cache), k_cache.shape[1], _ptr(pos), max_len, ws, nws,
                                               _stream(dev)))
        return y


def decode_layers(blocks: Sequence[QuantizedLLaMABlock], x: torch.Tensor, cache: KVCache, max_len: int,
                  out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """One decode step through a stack of blocks (the layer loop of
    NanoLLaMA::forward, models.hpp:257-266, for one new token per sequence).
    The first block reads x and every block writes the hidden state `out` in
    place.  Does not advance pos."""
    h = out if out is not None else torch.empty_like(x)
    src = x
    for i, blk in enumerate(blocks):
        blk.decode(src, cache.k[i], cache.v[i], cache.pos, max_len, out=h)
        src = h
    return h


def embedding(indices: torch.Tensor, weight: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """embedding (src/ops.cpp:2624-2650) on the device: fp32 token ids in, rows of weight out."""
    lib = load_library()
    idx = _dev_f32(indices).reshape(-1)
    w = _dev_f32(weight)
    y = out if out is not None else torch.empty((idx.numel(), w.shape[1]), dtype=torch.float32, device=w.device)
    _check(lib.sgq_embedding(_ptr(idx), idx.numel(), _ptr(w), w.shape[0], w.shape[1], _ptr(y), _stream(w.device)))
    return y


class QuantizedNanoLLaMA:
    """NanoLLaMA (include/sovereigngrad/models.hpp:226-303) with quantized
    blocks and an INT4 lm_head, decoding with a KV cache:

      h = token_embeddings(ids); h = layer(h) for each layer; h = norm_f(h);
      logits = lm_head(h)                                  (models.hpp:257-266)

    generate() follows NanoLLaMA::generate's greedy choice (models.hpp:270-302:
    softmax of logits / temperature, then the first index of the largest
    probability); the argmax of the logits is the same index, so the softmax is
    not formed."""

    def __init__(self, tok_emb: torch.Tensor, blocks: Sequence[QuantizedLLaMABlock], norm_f: torch.Tensor,
                 lm_head: QuantizedTensor, lm_bias: Optional[torch.Tensor] = None, eps: float = 1e-5):
        self.tok_emb = _dev_f32(tok_emb)
        self.blocks = list(blocks)
        self.norm_f = _dev_f32(norm_f).reshape(-1)
        self.lm_head, self.lm_bias, self.eps = lm_head, lm_bias, eps
        self.D = self.tok_emb.shape[1]
        self.V = lm_head.cols

    def new_cache(self, B: int, max_tokens: int) -> KVCache:
        return KVCache(B, max_tokens, self.D, self.tok_emb.device, layers=len(self.blocks))

    def step(self, token_ids: torch.Tensor, cache: KVCache, max_len: int) -> torch.Tensor:
        """One token per sequence (fp32 ids [B]) at positions cache.pos; returns
        logits [B, V].  The caller advances cache.pos."""
        from . import quantized_matmul_int4

        x = embedding(token_ids, self.tok_emb)
        h = decode_layers(self.blocks, x, cache, max_len)
        return quantized_matmul_int4(rms_norm(h, self.norm_f, self.eps), self.lm_head, self.lm_bias)

    def generate(self, prompts: Sequence[Sequence[int]], max_new_tokens: int) -> list:
        """Greedy continuation of each prompt (all prompts of one length), one
        decode step per token: the prompt is fed token by token, then each new
        token is chosen from the last logits."""
        B, L = len(prompts), len(prompts[0])
        if any(len(p) != L for p in prompts) or L == 0:
            raise ValueError("prompts must be non-empty and of one length")
        dev = self.tok_emb.device
        cache = self.new_cache(B, L + max_new_tokens)
        out = [list(p) for p in prompts]
        cur = torch.tensor([p[0] for p in prompts], dtype=torch.float32, device=dev)
        for t in range(L + max_new_tokens - 1):
            cache.pos.fill_(t)
            logits = self.step(cur, cache, t + 1)
            if t + 1 < L:
                cur = torch.tensor([p[t + 1] for p in prompts], dtype=torch.float32, device=dev)
                continue
            # The reference picks on the host, keeping the first maximum.
            nxt = logits.cpu().numpy().argmax(axis=1).tolist()
            for b in range(B):
                out[b].append(int(nxt[b]))
            cur = torch.tensor(nxt, dtype=torch.float32, device=dev)
        return out


__all__ = ["PROJECTIONS", "Int4Linear", "LlamaBlockInt4", "projection_shapes", "attention_scale", "rms_norm",
           "KVCache", "QuantizedLLaMABlock", "decode_layers", "embedding", "QuantizedNanoLLaMA"]
