"""Synthetic Qwen2-layout GPTQ int4 checkpoints for the loader tests (Python and Node hosts)."""
import numpy as np

from webllm_amd import gptq, synth

TINY = gptq.QwenConfig(vocab_size=512, block_size=16, n_layer=2, n_head=4, n_kv_head=2,
                       n_embd=256, intermediate=640)


def post_norm_weight(cfg, layer):
    """The post-attention RMSNorm weight of `layer` in these checkpoints: 1 + 0.1 N(0,1) per channel
    (the input norms are ones)."""
    return (1.0 + 0.1 * synth.activations(1, cfg.n_embd, seed=0x10AE, key=(layer,))[0]).astype(np.float32)


def write_checkpoint(path, cfg, act_order=None, no_g_idx=False):
    """Writes a Qwen-layout GPTQ checkpoint of config `cfg` (random tensors, half the linears with
    qzeros nibble 7, half with random zeros) and returns {(layer, key): (GptqTensors, bias f32)} plus "embed": the fp16 embedding.
    act_order=(layer, key): that linear gets a permuted g_idx (a desc_act=true checkpoint);
    no_g_idx: no g_idx tensors at all."""
    shapes = gptq.qwen_linear_shapes(cfg)
    tensors, kept = {}, {}
    rng = np.random.default_rng(1)
    emb = (rng.standard_normal((cfg.vocab_size, cfg.n_embd)) * 0.02).astype(np.float16)
    tensors["model.embed_tokens.weight"] = ("F16", emb.shape, emb.tobytes())
    kept["embed"] = emb
    tensors["model.norm.weight"] = ("F32", (cfg.n_embd,), np.ones(cfg.n_embd, np.float32).tobytes())
    for i in range(cfg.n_layer):
        p = f"model.layers.{i}"
        tensors[f"{p}.input_layernorm.weight"] = ("F32", (cfg.n_embd,), np.ones(cfg.n_embd, np.float32).tobytes())
        tensors[f"{p}.post_attention_layernorm.weight"] = ("F32", (cfg.n_embd,), post_norm_weight(cfg, i).tobytes())
        for j, (key, proj) in enumerate(gptq._PROJ):
            K, N = shapes[key]
            t = synth.gptq_linear(K, N, 128, seed=0x10AD, key=(i, j), stored_zero=None if j % 2 else 7)
            pre = f"{p}.{proj}"
            tensors[f"{pre}.qweight"] = ("I32", t.qweight.shape, t.qweight.tobytes())
            tensors[f"{pre}.qzeros"] = ("I32", t.qzeros.shape, t.qzeros.tobytes())
            tensors[f"{pre}.scales"] = ("F16", t.scales.shape, t.scales.tobytes())
            g_idx = (np.arange(K) // 128).astype(np.int32)
            if act_order == (i, key):
                g_idx = g_idx[np.random.default_rng(7).permutation(K)]
            if not no_g_idx:
                tensors[f"{pre}.g_idx"] = ("I32", g_idx.shape, g_idx.tobytes())
            b = None
            if key in gptq._BIASED:
                b = rng.standard_normal(N).astype(np.float16)
                tensors[f"{pre}.bias"] = ("F16", (N,), b.tobytes())
                b = b.astype(np.float32)
            kept[(i, key)] = (t, b)
    gptq.write_safetensors(path, tensors)
    return kept
