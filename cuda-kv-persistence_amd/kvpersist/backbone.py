"""Python mirror of the upstream K/V producer, over the C-ABI of include/kvp_producer.h.

``BackboneConfig`` and ``SelfAttentionBackbone`` keep the reference's names,
fields, validation and call form (reference: src/config.py:6-41,
src/backbone.py:36-67): ``model = SelfAttentionBackbone(cfg, seed=0)``, then
``hidden, kv_per_layer = model(latents)`` with one ``(k, v)`` pair per layer
of shape (b, heads, t, head_dim). Here k and v are views of token-major
[b*T, D] device buffers (element (b, h, t, d) at row b*T + t, column
h*128 + d), the layout the attention path and the arena consume;
``forward_token_major`` returns those buffers directly. All compute runs in
libkvpersist.so; torch only provides device memory.

``layer_norm``, ``linear`` and ``qkv_project`` expose the block's pieces
(nn.LayerNorm, nn.Linear, the qkv_proj split; reference: src/backbone.py:13-34).
"""

from __future__ import annotations

import ctypes
import json
import secrets
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

from . import _lib
from .api import BF16, FP32, HEAD_DIM, _check, _ptr

_DT = {FP32: torch.float32, BF16: torch.bfloat16}


def _dtype_code(dtype) -> int:
    if dtype in (FP32, "fp32", torch.float32):
        return FP32
    if dtype in (BF16, "bf16", torch.bfloat16):
        return BF16
    raise ValueError(f"unsupported dtype {dtype!r} (fp32 or bf16)")


def _code_of(t: torch.Tensor) -> int:
    return _dtype_code(t.dtype)


@dataclass(frozen=True)
class BackboneConfig:
    """Reference: src/config.py:6-27 (same fields, defaults and checks)."""
    num_layers: int = 30
    hidden_dim: int = 1536
    num_heads: int = 12
    head_dim: int = 128
    latent_channels: int = 16
    tokens_per_frame: int = 1560
    latent_grid_rows: int = 30
    latent_grid_cols: int = 52
    tile_size_tokens: int = 16

    def __post_init__(self):
        if self.hidden_dim != self.num_heads * self.head_dim:
            raise ValueError(f"hidden_dim {self.hidden_dim} != num_heads({self.num_heads}) * "
                             f"head_dim({self.head_dim})")
        if self.latent_grid_rows * self.latent_grid_cols != self.tokens_per_frame:
            raise ValueError(f"latent grid {self.latent_grid_rows}x{self.latent_grid_cols} "
                             f"!= tokens_per_frame {self.tokens_per_frame}")

    @classmethod
    def from_grounding(cls, path="configs/grounding_config.json"):
        """Reference: src/config.py:29-41 (the "model" block of the grounding config)."""
        m = json.loads(Path(path).read_text())["model"]
        return cls(num_layers=m["layers"], hidden_dim=m["hidden_dim"], num_heads=m["heads"],
                   head_dim=m["head_dim"], tokens_per_frame=m["tokens_per_frame"],
                   latent_grid_rows=m["latent_grid"][0], latent_grid_cols=m["latent_grid"][1],
                   tile_size_tokens=m["tile_size_tokens"])


def layer_norm(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, out: torch.Tensor,
               eps: float = 1e-5, stream: int | None = None) -> torch.Tensor:
    """out = LayerNorm(x) over the last dim; weight/bias fp32."""
    D = x.shape[-1]
    _check(_lib.load().kvp_layer_norm(_code_of(x), _code_of(out), _ptr(x), _ptr(weight),
                                      _ptr(bias), _ptr(out), x.numel() // D, D, eps, stream),
           "kvp_layer_norm")
    return out


def linear(x: torch.Tensor, weight, bias, out: torch.Tensor, accumulate: bool = False,
           stream: int | None = None) -> torch.Tensor:
    """out (+)= x weight^T + bias; weight [out, in] in x's dtype, bias fp32 [out]
    or None (tensors or device addresses); the sizes come from x and out."""
    n_in = x.shape[-1]
    n_out = out.shape[-1]
    _check(_lib.load().kvp_linear(_code_of(x), _code_of(out), _ptr(x), _ptr(weight), _ptr(bias),
                                  _ptr(out), x.numel() // n_in, n_in, n_out, int(accumulate),
                                  stream), "kvp_linear")
    return out


def proj_gemm(x: torch.Tensor, weight, bias, outs, accumulate: bool = False, tile_n: int = 128,
              stream: int | None = None) -> None:
    """Grouped projection on the hand-written kernel: outs[g] (+)= x W_g^T + b_g
    with W_g the g-th [N]-row block of weight (bf16) and N = outs[0].shape[-1]."""
    outs = list(outs)
    n = outs[0].shape[-1]
    k = x.shape[-1]
    ptrs = [_ptr(o) for o in outs] + [None] * (3 - len(outs))
    _check(_lib.load().kvp_proj_gemm(_ptr(x), _ptr(weight), _ptr(bias), ptrs[0], ptrs[1],
                                     ptrs[2], len(outs), x.numel() // k, k, n,
                                     _code_of(outs[0]), int(accumulate), tile_n, stream),
           "kvp_proj_gemm")


def qkv_project(x: torch.Tensor, ln_weight, ln_bias, qkv_weight, qkv_bias, xn, q, k, v,
                stream: int | None = None) -> None:
    """LN(x) then q, k, v = the three [D]-row blocks of qkv_proj (x fp32 [rows, D])."""
    D = x.shape[-1]
    _check(_lib.load().kvp_qkv_project(_code_of(q), _ptr(x), _ptr(ln_weight), _ptr(ln_bias),
                                       _ptr(qkv_weight), _ptr(qkv_bias), _ptr(xn), _ptr(q),
                                       _ptr(k), _ptr(v), x.numel() // D, D, stream),
           "kvp_qkv_project")


class SelfAttentionBackbone:
    """Reference: src/backbone.py:36-67, on libkvpersist.so.

    ``init`` must be "random" (the reference raises NotImplementedError for
    anything else; weights can be loaded with ``load_state_dict``). ``seed``
    None draws a fresh seed. Parameters are initialised on the device with
    the reference's distributions from this library's own generator."""

    def __init__(self, cfg: BackboneConfig | None = None, init: str = "random",
                 seed: int | None = None, dtype="fp32"):
        if init != "random":
            raise NotImplementedError("pretrained weights: use load_state_dict")
        self.cfg = cfg or BackboneConfig()
        if self.cfg.head_dim != HEAD_DIM:
            raise ValueError(f"head_dim must be {HEAD_DIM} (the attention kernels' head size)")
        self.dtype = _dtype_code(dtype)
        self.seed = secrets.randbits(63) if seed is None else int(seed)
        self._lib = _lib.load()
        c = self.cfg
        self._h = self._lib.kvp_backbone_create(self.dtype, c.num_layers, c.tokens_per_frame,
                                                c.hidden_dim, c.num_heads, c.latent_channels,
                                                self.seed & 0xFFFFFFFFFFFFFFFF)
        if not self._h:
            raise RuntimeError(f"kvp_backbone_create failed: {_lib.last_error()}")

    def close(self):
        if getattr(self, "_h", None):
            self._lib.kvp_backbone_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    # ---- parameters -------------------------------------------------------
    def param_count(self) -> int:
        return int(self._lib.kvp_backbone_param_count(self._h))

    def param_names(self) -> list[str]:
        n = self._lib.kvp_backbone_num_tensors(self._h)
        return [self._lib.kvp_backbone_tensor_name(self._h, i).decode() for i in range(n)]

    def param_info(self, name: str) -> tuple[int, int, int]:
        """(device address, numel, dtype code) of a named parameter."""
        ptr = ctypes.c_void_p()
        numel = ctypes.c_long()
        dt = ctypes.c_int()
        _check(self._lib.kvp_backbone_param_info(self._h, name.encode(), ctypes.byref(ptr),
                                                 ctypes.byref(numel), ctypes.byref(dt)),
               f"param_info({name})")
        return int(ptr.value or 0), int(numel.value), int(dt.value)

    def _shape(self, name: str) -> tuple[int, ...]:
        D, C = self.cfg.hidden_dim, self.cfg.latent_channels
        if name == "token_embed.weight":
            return (D, C)
        if name.endswith("qkv_proj.weight"):
            return (3 * D, D)
        if name.endswith("qkv_proj.bias"):
            return (3 * D,)
        if name.endswith("out_proj.weight"):
            return (D, D)
        return (D,)

    def get_param(self, name: str) -> torch.Tensor:
        """fp32 CPU copy of a parameter, in the reference's shape."""
        _, numel, _ = self.param_info(name)
        host = np.empty(numel, dtype=np.float32)
        _check(self._lib.kvp_backbone_get_param(self._h, name.encode(),
                                                host.ctypes.data_as(_lib.c_float_p), numel),
               f"get_param({name})")
        return torch.from_numpy(host).view(self._shape(name))

    def set_param(self, name: str, value) -> None:
        host = np.ascontiguousarray(np.asarray(value, dtype=np.float32).reshape(-1))
        _check(self._lib.kvp_backbone_set_param(self._h, name.encode(),
                                                host.ctypes.data_as(_lib.c_float_p), host.size),
               f"set_param({name})")

    def state_dict(self) -> dict[str, torch.Tensor]:
        return {n: self.get_param(n) for n in self.param_names()}

    def load_state_dict(self, sd) -> None:
        names = self.param_names()
        missing = [n for n in names if n not in sd]
        unexpected = [n for n in sd if n not in names]
        if missing or unexpected:
            raise KeyError(f"missing {missing[:4]} unexpected {unexpected[:4]}")
        for n in names:
            t = sd[n]
            self.set_param(n, t.detach().float().cpu().numpy() if isinstance(t, torch.Tensor)
                           else t)

    # ---- forward ----------------------------------------------------------
    def forward_token_major(self, latents: torch.Tensor, keep_q: bool = False,
                            stream: int | None = None):
        """latents (b, C, rows, cols) or (b, C*T) fp32 on the device ->
        (hidden [b*T, D] fp32, k [L, b*T, D], v [L, b*T, D], q or None)."""
        c = self.cfg
        if latents.dtype != torch.float32 or not latents.is_cuda:
            raise ValueError("latents must be a float32 device tensor")
        lat = latents.contiguous()
        b = lat.shape[0]
        if lat.numel() != b * c.latent_channels * c.tokens_per_frame:
            raise ValueError(f"latents hold {lat.numel()} values, expected "
                             f"b * {c.latent_channels} * {c.tokens_per_frame}")
        rows = b * c.tokens_per_frame
        dev = lat.device
        dt = _DT[self.dtype]
        hidden = torch.empty(rows, c.hidden_dim, dtype=torch.float32, device=dev)
        k = torch.empty(c.num_layers, rows, c.hidden_dim, dtype=dt, device=dev)
        v = torch.empty_like(k)
        q = torch.empty_like(k) if keep_q else None
        _check(self._lib.kvp_backbone_forward(self._h, _ptr(lat), b, _ptr(hidden), _ptr(q),
                                              _ptr(k), _ptr(v), rows * c.hidden_dim, stream),
               "backbone forward")
        return hidden, k, v, q

    def forward(self, latents: torch.Tensor, timestep=None, context=None):
        """Reference signature: (hidden (b, T, D), [(k, v)] with k, v (b, heads, T, hd))."""
        del timestep, context
        c = self.cfg
        b = latents.shape[0]
        hidden, k, v, _ = self.forward_token_major(latents)
        shape = (b, c.tokens_per_frame, c.num_heads, c.head_dim)
        kv = [(k[i].view(shape).permute(0, 2, 1, 3), v[i].view(shape).permute(0, 2, 1, 3))
              for i in range(c.num_layers)]
        return hidden.view(b, c.tokens_per_frame, c.hidden_dim), kv

    __call__ = forward
