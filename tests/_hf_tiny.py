"""A tiny random-initialised Qwen3-VL text decoder with an untied vocabulary head
(the structure the reference's patch walks), for the integration-shim tests."""
import torch
import torch.nn as nn


def tiny_config(hidden=256, ffn=512, layers=2, heads=4, kv_heads=2, head_dim=64, vocab=1024):
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLTextConfig
    cfg = Qwen3VLTextConfig(hidden_size=hidden, intermediate_size=ffn, num_hidden_layers=layers,
                            num_attention_heads=heads, num_key_value_heads=kv_heads, head_dim=head_dim,
                            vocab_size=vocab,
                            rope_scaling={"rope_type": "default", "mrope_section": [16, 8, 8],
                                          "mrope_interleaved": True, "rope_theta": 1e6})
    cfg._attn_implementation = "sdpa"
    return cfg


class Out:
    def __init__(self, logits, past_key_values):
        self.logits, self.past_key_values = logits, past_key_values


class TinyLM(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLTextModel
        self.model = Qwen3VLTextModel(cfg)
        self.lm_head = nn.Linear(cfg.hidden_size, cfg.vocab_size, bias=False)

    def forward(self, input_ids, position_ids=None, attention_mask=None, past_key_values=None, use_cache=True):
        h = self.model(input_ids=input_ids, position_ids=position_ids, attention_mask=attention_mask,
                       past_key_values=past_key_values, use_cache=use_cache).last_hidden_state
        return Out(self.lm_head(h), past_key_values)


def tiny_model(seed=0, device="cpu", **kw):
    torch.manual_seed(seed)
    m = TinyLM(tiny_config(**kw))
    with torch.no_grad():
        for p in m.parameters():
            if p.dim() == 1:        # RMSNorm weights: 1 + N(0, 0.02) instead of ones
                p.copy_(1 + 0.02 * torch.randn_like(p))
    return m.to(device=device, dtype=torch.bfloat16).eval()
