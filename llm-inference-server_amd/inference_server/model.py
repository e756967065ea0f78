"""GPT-2 for the end-to-end configs: the reference architecture with seeded random
weights.

The reference loads pretrained `gpt2` from the hub by name (inference_server/model.py:
18-33); there is no network here, so the model is `GPT2LMHeadModel(GPT2Config())`
initialised after seeding with SEED (config.py:16) — the same 124M architecture
(12 layers, 12 heads, head_dim 64, vocab 50257). Workloads supply token ids directly;
no tokenizer is needed. `small=True` builds a 2-layer variant for CPU tests.
"""

from __future__ import annotations

import torch
from transformers import GPT2Config, GPT2LMHeadModel

from inference_server.config import SEED, seed_everything

EOS_TOKEN_ID = 50256  # GPT-2's <|endoftext|>


class NoTokenizer:
    """What the executor and engine need of a tokenizer when ids are fed directly."""

    def __init__(self, eos_token_id: int = EOS_TOKEN_ID) -> None:
        self.eos_token_id = eos_token_id

    def decode(self, ids, skip_special_tokens=True) -> str:
        return " ".join(str(i) for i in ids)


def load(dtype: torch.dtype = torch.float32, device: str = "cpu", small: bool = False, seed: int = SEED):
    seed_everything(seed)
    if small:
        cfg = GPT2Config(n_layer=2, n_head=4, n_embd=128, vocab_size=1000, n_positions=512,
                         bos_token_id=999, eos_token_id=999)
    else:
        cfg = GPT2Config()
    model = GPT2LMHeadModel(cfg)
    model.to(dtype=dtype, device=device)
    model.eval()
    return model, NoTokenizer(cfg.eos_token_id)


def sync(device: str) -> None:
    if torch.device(device).type == "cuda":
        torch.cuda.synchronize()
