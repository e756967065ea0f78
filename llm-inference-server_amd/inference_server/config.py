"""Process-wide configuration read from the environment, mirroring the reference's
`Config` (inference_server/config.py:54-109) for the fields the paged-KV path reads.

`attention` is the backend switch of core/attention.py. The reference knows `gather`
and `triton`; this build adds `hip`, which routes attention, the KV append, block
copy and swap through libpagedkv's CDNA4 kernels and never falls back.
"""

from __future__ import annotations

import os
import random
from dataclasses import dataclass, field

import numpy as np
import torch

SEED = 1337                      # config.py:16
DEFAULT_NUM_BLOCKS = 2048        # config.py:20: max_running * max_seq_len / block_size
ATTENTION_BACKENDS = ("gather", "triton", "hip")


def seed_everything(seed: int = SEED) -> None:
    random.seed(seed)
    np.random.seed(seed)
    torch.manual_seed(seed)


def pick_device() -> str:
    """DEVICE if set, else cuda (ROCm reports itself as cuda) when a GPU is visible."""
    if forced := os.environ.get("DEVICE"):
        return forced
    return "cuda" if torch.cuda.is_available() else "cpu"


@dataclass
class Config:
    device: str = field(default_factory=pick_device)
    dtype: str = os.environ.get("DTYPE", "float32")

    max_running: int = int(os.environ.get("MAX_RUNNING", 32))
    max_queue_depth: int = 256

    block_size: int = int(os.environ.get("BLOCK_SIZE", 16))
    num_blocks: int = int(os.environ.get("NUM_BLOCKS", DEFAULT_NUM_BLOCKS))
    attention: str = os.environ.get("ATTENTION", "gather")
    prefix_caching: bool = os.environ.get("PREFIX_CACHING", "1") == "1"
    preemption: str = os.environ.get("PREEMPTION", "recompute")
    # ATTENTION=hip on a GPU: replay decode steps as captured HIP graphs (one per batch size),
    # and prefill steps too (one per packed-token bucket) unless PREFILL_GRAPHS=0.
    decode_graphs: bool = os.environ.get("DECODE_GRAPHS", "1") == "1"
    prefill_graphs: bool = os.environ.get("PREFILL_GRAPHS", "1") == "1"
    # ATTENTION=hip with an fp16/bf16 model: greedy ids straight from the LM head
    # (pkv_lm_head_argmax) instead of logits + argmax, unless FUSED_GREEDY=0.
    fused_greedy: bool = os.environ.get("FUSED_GREEDY", "1") == "1"
    # ATTENTION=hip, fp16/bf16 pool: each layer's KV append happens inside the attention
    # call (decode and prefill steps), unless FUSED_APPEND=0.
    fused_append: bool = os.environ.get("FUSED_APPEND", "1") == "1"
    # ATTENTION=hip, fp16/bf16 GPT-2-style model (a fused QKV Conv1D): decode steps
    # project Q/K/V with pkv_qkv_append, which stores K and V at their pool slots in its
    # epilogue (faster than the model's hipBLASLt GEMM at decode batch sizes on MI355X),
    # unless QKV_EPILOGUE=0.
    qkv_epilogue: bool = os.environ.get("QKV_EPILOGUE", "1") == "1"

    default_max_tokens: int = 128
    max_seq_len: int = 1024

    @property
    def torch_dtype(self) -> torch.dtype:
        return {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}[self.dtype]

    @property
    def kv_backend(self) -> str:
        """Which kernels move KV bytes (append / copy / swap): the HIP library when
        ATTENTION=hip, torch ops (the reference's own calls) otherwise."""
        return "hip" if self.attention == "hip" else "torch"


CONFIG = Config()
