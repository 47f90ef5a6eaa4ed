"""Model shapes of the synthetic qwen35 models the tests and the benchmark use.

Q4_K_M-style quantization: Q6_K for the LM head, attn_v and ffn_down, Q4_K for
every other matrix (token embedding, ssm_beta/alpha and ssm_out included);
norms, conv1d, dt and A stay F32 as the loader requires. Values: matrices
N(0, 0.02), norm weights 1 + 0.1 N, ssm_a = -exp(0.5 N), ssm_dt and conv1d
0.5 N, all from the library's seeded generator (base seed 20261107).
"""
from dataclasses import dataclass, replace

F32, Q8_0, Q4_K, Q6_K = 0, 8, 12, 14
BASE_SEED = 20261107


@dataclass(frozen=True)
class SynthConfig:
    n_layer: int
    n_embd: int
    n_ff: int
    n_vocab: int
    n_head: int
    n_head_kv: int
    head_dim: int
    n_rot: int
    rope_base: float = 1e7
    eps: float = 1e-6
    conv_k: int = 4
    s_k: int = 128
    h_k: int = 16
    h_v: int = 16
    full_attn_interval: int = 4
    type_default: int = Q4_K
    type_embd: int = Q4_K
    type_out: int = Q6_K
    type_v: int = Q6_K
    type_down: int = Q6_K
    w_std: float = 0.02
    seed: int = BASE_SEED
    nextn: int = 0        # 1: one MTP layer after the main layers
    eos_id: int = -1      # >= 0: tokenizer.ggml.eos_token_id
    eot_id: int = -1      # >= 0: a token list with "<|im_end|>" at this id

    def with_(self, **kw):
        return replace(self, **kw)

    def weight_bytes_per_token(self):
        """HBM bytes of the weights one decode step reads (every layer + LM head, not the embedding)."""
        from . import row_bytes
        E, FF, V, H, Hk, D = self.n_embd, self.n_ff, self.n_vocab, self.n_head, self.n_head_kv, self.head_dim
        DI, KD = self.h_v * self.s_k, self.h_k * self.s_k
        CD = 2 * KD + DI
        t, b = self.type_default, 0
        for i in range(self.n_layer):
            b += 2 * FF * row_bytes(t, E) + E * row_bytes(self.type_down, FF)
            if (i + 1) % self.full_attn_interval:
                b += (CD + DI + 2 * self.h_v) * row_bytes(t, E) + E * row_bytes(t, DI)
                b += 4 * (CD * self.conv_k + 2 * self.h_v + self.s_k)
            else:
                b += (2 * H * D + Hk * D) * row_bytes(t, E) + Hk * D * row_bytes(self.type_v, E)
                b += E * row_bytes(t, H * D) + 8 * D
            b += 8 * E
        return b + V * row_bytes(self.type_out, E) + 4 * E


# 0.8B shape: hidden 1024, 24 layers (18 DeltaNet + 6 GQA), GQA 8q/2kv d=256, FFN 3584
CONFIG_0_8B = SynthConfig(n_layer=24, n_embd=1024, n_ff=3584, n_vocab=151936, n_head=8, n_head_kv=2,
                          head_dim=256, n_rot=64, s_k=128, h_k=16, h_v=16)
# 4B shape: hidden 2560, 32 layers (24 DeltaNet + 8 GQA), DeltaNet 32 heads d=128, GQA 16q/4kv d=256, FFN 9216
CONFIG_4B = SynthConfig(n_layer=32, n_embd=2560, n_ff=9216, n_vocab=151936, n_head=16, n_head_kv=4,
                        head_dim=256, n_rot=64, s_k=128, h_k=32, h_v=32, seed=BASE_SEED + 4)
# small models with the same structure for parity tests (value heads a multiple of key heads)
TINY = SynthConfig(n_layer=8, n_embd=256, n_ff=512, n_vocab=2048, n_head=2, n_head_kv=1, head_dim=128, n_rot=32,
                   rope_base=1e4, s_k=64, h_k=2, h_v=4, w_std=0.05, seed=BASE_SEED + 1)
# the tiny model with an MTP layer (the main layers' weights are those of TINY)
TINY_MTP = SynthConfig(n_layer=8, n_embd=256, n_ff=512, n_vocab=2048, n_head=2, n_head_kv=1, head_dim=128, n_rot=32,
                       rope_base=1e4, s_k=64, h_k=2, h_v=4, w_std=0.05, seed=BASE_SEED + 1, nextn=1)
# the 0.8B shape with an MTP layer
CONFIG_0_8B_MTP = CONFIG_0_8B.with_(nextn=1)
TINY_DRAFT = SynthConfig(n_layer=4, n_embd=256, n_ff=512, n_vocab=2048, n_head=2, n_head_kv=1, head_dim=128,
                         n_rot=32, rope_base=1e4, s_k=64, h_k=4, h_v=4, w_std=0.05, seed=BASE_SEED + 2)
