# Type stubs of fusedtok_amd's public API (PEP 561; the package ships
# py.typed). Names, parameters and defaults follow the fusedtok 2.5.0 decode
# hot path (reference python/fusedtok/__init__.pyi:99-107,208-236); the
# build's additions are the extra keywords and the fused / test-hook ops.

from typing import List, Optional, Sequence, Tuple, Union, overload

import numpy as np
import torch

Array = Union[np.ndarray, torch.Tensor]
IntArray = Union[np.ndarray, torch.Tensor, Sequence[int]]
Scale = Union[float, torch.Tensor]
Histories = Union[np.ndarray, torch.Tensor, Sequence[Sequence[int]]]

__version__: str

__all__ = [
    "cuda_available",
    "rmsnorm",
    "rope",
    "swiglu",
    "quantize_int8",
    "dequantize_int8",
    "qadd_int8",
    "qgemm",
    "qgemm_perchannel",
    "qgemm_i32",
    "attention_decode",
    "attention_decode_paged",
    "attention_decode_paged_quant",
    "attention_decode_paged_append",
    "attention_prefill",
    "kv_append",
    "kv_append_paged",
    "rmsnorm_quant",
    "rmsnorm_qgemm",
    "swiglu_quant",
    "rope_kv_append_paged",
    "qgemm_rope_kv_append_paged",
    "qgemm_rmsnorm_quant",
    "qgemm_swiglu_quant",
    "DecodeLayer",
    "DecodeStack",
    "argmax",
    "argmax_batched",
    "sample_topp",
    "sample_topp_batched",
    "decode_step",
    "decode_step_batched",
]

def cuda_available() -> bool: ...

# -- elementwise / row ops ---------------------------------------------------
def swiglu(gate: Array, up: Array, *, cuda: bool = ...) -> Array: ...
def rmsnorm(x: Array, weight: Array, *, residual: Optional[Array] = ...,
            eps: float = ..., cuda: bool = ...) -> Array: ...
def rope(q: Array, k: Optional[Array] = ..., *, theta: float = ...,
         pos_offset: int = ..., neox: bool = ..., cuda: bool = ...,
         positions: Optional[torch.Tensor] = ...,
         rows_per_position: int = ...) -> Tuple[Array, Optional[Array]]: ...

# -- attention -----------------------------------------------------------------
def attention_decode(q: Array, k_cache: Array, v_cache: Array,
                     lens: Optional[IntArray] = ..., *, cuda: bool = ...) -> Array: ...
def attention_decode_paged(q: Array, k_pool: Array, v_pool: Array,
                           block_table: IntArray, lens: Optional[IntArray] = ..., *,
                           cuda: bool = ...) -> Array: ...
def attention_decode_paged_quant(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                                 block_table: torch.Tensor,
                                 lens: Optional[torch.Tensor] = ..., *,
                                 device_scale: bool = ...
                                 ) -> Tuple[torch.Tensor, torch.Tensor, Scale]: ...
def attention_decode_paged_append(q: torch.Tensor, k_pool: torch.Tensor,
                                  v_pool: torch.Tensor, block_table: torch.Tensor,
                                  k_new: torch.Tensor, v_new: torch.Tensor,
                                  lens: torch.Tensor) -> torch.Tensor: ...
def attention_prefill(q: Array, k: Array, v: Array, causal: bool = ..., *,
                      cuda: bool = ...) -> Array: ...
def kv_append(k_cache: Array, v_cache: Array, k_new: Array, v_new: Array,
              lens: IntArray, *, cuda: bool = ...) -> None: ...
def kv_append_paged(k_pool: Array, v_pool: Array, block_table: IntArray,
                    k_new: Array, v_new: Array, lens: IntArray, *,
                    cuda: bool = ...) -> None: ...

# -- int8 ------------------------------------------------------------------------
@overload
def quantize_int8(x: Array) -> Tuple[Array, float]: ...
@overload
def quantize_int8(x: Array, *, device_scale: bool) -> Tuple[Array, Scale]: ...
def dequantize_int8(q: Array, scale: Scale, *,
                    out_dtype: Optional[torch.dtype] = ...) -> Array: ...
def qadd_int8(qa: torch.Tensor, sa: Scale, qb: torch.Tensor, sb: Scale, *,
              device_scale: bool = ...) -> Tuple[torch.Tensor, Scale]: ...
def qgemm(a_q: Array, a_scale: Scale, b_q: Array, b_scale: float, *,
          cuda: bool = ..., out_dtype: Optional[torch.dtype] = ...) -> Array: ...
def qgemm_perchannel(a_q: Array, a_scale: Scale, b_q: Array,
                     b_scales: Union[Array, Sequence[float]], *, cuda: bool = ...,
                     out_dtype: Optional[torch.dtype] = ...) -> Array: ...
def qgemm_i32(a_q: Array, b_q: Array) -> Array: ...

# -- fused decode-chain steps (GPU tensors only) -------------------------------
def rmsnorm_quant(x: torch.Tensor, weight: torch.Tensor, *,
                  residual: Optional[torch.Tensor] = ..., eps: float = ...,
                  device_scale: bool = ...) -> Tuple[torch.Tensor, Scale]: ...
def rmsnorm_qgemm(x: torch.Tensor, weight: torch.Tensor, b_q: torch.Tensor,
                  b_scales: Union[torch.Tensor, Sequence[float], float], *,
                  residual: Optional[torch.Tensor] = ..., eps: float = ...,
                  out_dtype: Optional[torch.dtype] = ...
                  ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]: ...
def swiglu_quant(gate: torch.Tensor, up: torch.Tensor, *,
                 device_scale: bool = ...) -> Tuple[torch.Tensor, Scale]: ...
def rope_kv_append_paged(qkv: torch.Tensor, q_heads: int, kv_heads: int,
                         k_pool: torch.Tensor, v_pool: torch.Tensor,
                         block_table: IntArray, lens: IntArray, *,
                         theta: float = ..., pos_offset: int = ...,
                         neox: bool = ...) -> torch.Tensor: ...
def qgemm_rope_kv_append_paged(a_q: torch.Tensor, a_scale: Scale, w_q: torch.Tensor,
                               w_scales: Union[torch.Tensor, Sequence[float]], q_heads: int,
                               kv_heads: int, k_pool: torch.Tensor, v_pool: torch.Tensor,
                               block_table: IntArray, lens: IntArray, *, theta: float = ...,
                               pos_offset: int = ..., neox: bool = ...
                               ) -> Tuple[torch.Tensor, torch.Tensor]: ...
def qgemm_rmsnorm_quant(a_q: torch.Tensor, a_scale: Scale, w_q: torch.Tensor,
                        w_scales: Union[torch.Tensor, Sequence[float]], weight: Array, *,
                        residual: Optional[torch.Tensor] = ..., eps: float = ...,
                        out_dtype: Optional[torch.dtype] = ..., device_scale: bool = ...
                        ) -> Tuple[torch.Tensor, torch.Tensor, Scale]: ...
def qgemm_swiglu_quant(a_q: torch.Tensor, a_scale: Scale, w_q: torch.Tensor,
                       w_scales: Union[torch.Tensor, Sequence[float]], *,
                       out_dtype: Optional[torch.dtype] = ..., device_scale: bool = ...
                       ) -> Tuple[torch.Tensor, torch.Tensor, Scale]: ...

# -- post-logits sampling -------------------------------------------------------
def argmax(x: Array, *, cuda: bool = ...) -> int: ...
def argmax_batched(x: Array, *, cuda: bool = ...) -> Array: ...
def sample_topp(logits: Array, p: float, *, temperature: float = ..., seed: int = ...,
                cuda: bool = ...) -> int: ...
def sample_topp_batched(logits: Array, p: float, *, temperature: float = ...,
                        seeds: Optional[IntArray] = ..., cuda: bool = ...,
                        device_out: bool = ...) -> Array: ...
def decode_step(logits: Array, sampled_ids: IntArray, penalty: float = ..., *,
                p: float = ..., temperature: float = ..., seed: int = ...,
                cuda: bool = ...) -> int: ...
def decode_step_batched(logits: Array, sampled_ids: Histories, penalty: float = ..., *,
                        p: float = ..., temperature: float = ...,
                        seeds: Optional[IntArray] = ...,
                        ids_offsets: Optional[IntArray] = ..., cuda: bool = ...,
                        device_out: bool = ...) -> Array: ...

class DecodeLayer:
    hidden: int
    q_heads: int
    kv_heads: int
    head_dim: int
    inter: int
    page: int
    max_batch: int
    dtype: torch.dtype
    def __init__(self, *, norm1: torch.Tensor, w_qkv: torch.Tensor, s_qkv: torch.Tensor,
                 w_o: torch.Tensor, s_o: torch.Tensor, norm2: torch.Tensor,
                 w_gu: torch.Tensor, s_gu: torch.Tensor, w_down: torch.Tensor,
                 s_down: torch.Tensor, q_heads: int, kv_heads: int, page: int,
                 max_batch: int, dtype: torch.dtype = ..., eps: float = ...,
                 theta: float = ..., neox: bool = ..., pos_offset: int = ...) -> None: ...
    def forward(self, x: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                block_table: torch.Tensor, lens: torch.Tensor, *,
                out: Optional[torch.Tensor] = ...) -> torch.Tensor: ...
    def __call__(self, x: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                 block_table: torch.Tensor, lens: torch.Tensor, *,
                 out: Optional[torch.Tensor] = ...) -> torch.Tensor: ...
    def capture(self, x: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                block_table: torch.Tensor, lens: torch.Tensor, *,
                out: Optional[torch.Tensor] = ...) -> torch.Tensor: ...
    def replay(self) -> torch.Tensor: ...
    def close(self) -> None: ...

class DecodeStack:
    layers: List[DecodeLayer]
    hidden: int
    max_batch: int
    dtype: torch.dtype
    def __init__(self, layers: Sequence[DecodeLayer]) -> None: ...
    def forward(self, x: torch.Tensor, k_pools: Sequence[torch.Tensor],
                v_pools: Sequence[torch.Tensor], block_table: torch.Tensor,
                lens: torch.Tensor, *, out: Optional[torch.Tensor] = ...) -> torch.Tensor: ...
    def __call__(self, x: torch.Tensor, k_pools: Sequence[torch.Tensor],
                 v_pools: Sequence[torch.Tensor], block_table: torch.Tensor,
                 lens: torch.Tensor, *, out: Optional[torch.Tensor] = ...) -> torch.Tensor: ...
    def capture(self, x: torch.Tensor, k_pools: Sequence[torch.Tensor],
                v_pools: Sequence[torch.Tensor], block_table: torch.Tensor,
                lens: torch.Tensor, *, out: Optional[torch.Tensor] = ...) -> torch.Tensor: ...
    def replay(self) -> torch.Tensor: ...
    def close(self) -> None: ...
