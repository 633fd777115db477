"""Tiny randomly initialised Llama models and a stub tokenizer for the runtime
tests (the reference's tests use the same geometry: vocab 256, hidden 64,
4 query / 2 KV heads, eos 1 -- tests/python/conftest.py:25-47)."""

from __future__ import annotations

from typing import List, Optional

import torch

VOCAB_SIZE = 256


def tiny_llama(num_layers: int = 2, seed: int = 0, device="cuda:0", dtype=torch.float32,
               head_dim: Optional[int] = None, hidden: int = 64, heads: int = 4, kv_heads: int = 2):
    from transformers import LlamaConfig, LlamaForCausalLM

    torch.manual_seed(seed)
    kwargs = {}
    if head_dim is not None:
        kwargs["head_dim"] = head_dim
    config = LlamaConfig(vocab_size=VOCAB_SIZE, hidden_size=hidden, intermediate_size=2 * hidden,
                         num_hidden_layers=num_layers, num_attention_heads=heads, num_key_value_heads=kv_heads,
                         max_position_embeddings=1024, eos_token_id=1, bos_token_id=0, pad_token_id=0, **kwargs)
    model = LlamaForCausalLM(config).to(device=device, dtype=dtype)
    model.eval()
    return model


class StubTokenizer:
    """Character tokenizer: ids 2..255 from characters, decode to letters."""

    eos_token_id = 1
    pad_token_id = 0
    chat_template = None

    def __call__(self, text, return_tensors=None):
        ids = [(ord(c) % (VOCAB_SIZE - 2)) + 2 for c in text] or [2]
        if return_tensors == "pt":
            return {"input_ids": torch.tensor([ids], dtype=torch.long)}
        return {"input_ids": ids}

    def decode(self, ids, skip_special_tokens=True):
        return "".join(chr((int(i) % 26) + 97) for i in ids)


@torch.no_grad()
def hf_greedy(model, prompt_ids: List[int], max_new_tokens: int, eos_ids=(1,), stop_on_eos: bool = True) -> List[int]:
    """Plain transformers greedy decoding with its own DynamicCache and its
    default attention: the engine's end-to-end oracle."""
    from transformers.cache_utils import DynamicCache

    device = next(model.parameters()).device
    cache = DynamicCache()
    ids = torch.tensor([prompt_ids], dtype=torch.long, device=device)
    out = model(input_ids=ids, past_key_values=cache, use_cache=True)
    generated: List[int] = []
    while True:
        tok = int(out.logits[0, -1].float().argmax())
        generated.append(tok)
        if (stop_on_eos and tok in eos_ids) or len(generated) >= max_new_tokens:
            return generated
        out = model(input_ids=torch.tensor([[tok]], dtype=torch.long, device=device), past_key_values=cache,
                    use_cache=True)
