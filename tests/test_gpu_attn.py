"""GPU parity of the decode attention over the KV cache and of the cache store (qwen.ts:424-442,
attention/attention_gqa_cache.wgsl, misc/kv_store.wgsl) against the oracle's attentionGqaRef
restatement (reference/qwen-ref.ts:65-111). Decode shapes (few rows x heads) split the keys over
workgroups and merge the splits in a second kernel; the cases cover one split and 10 to 128, runs
of 1 to 8 heads sharing a kv head, head dims 16 to 256 and a plan that the split workspace caps. Bar: the reference's own attention
tolerance, 1e-4
(tests/kernels.ts:1115), applied here as |got - ref| <= 1e-5 + 1e-4 |ref|; the cache store is a
copy and is bit-exact."""
import sys

import numpy as np
import pytest

from webllm_amd import gptq

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-5, 1e-4


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


CASES = [
    # (M, H, KV, D, past, max_t, heads per run, key splits, label): the plan is asserted
    (1, 14, 2, 64, 0, 128, 1, 1, "0.5B decode, first position"),
    (1, 14, 2, 64, 127, 128, 1, 1, "0.5B decode, full 128-position cache"),
    (16, 14, 2, 64, 100, 128, 1, 1, "16 rows over a cache (prefill continuation), causal"),
    (1, 28, 4, 128, 4095, 4096, 7, 64, "7B decode, 4096 positions: 64 key splits"),
    (1, 28, 4, 128, 8191, 8192, 7, 128, "7B decode, 8192 positions: 128 key splits (merge reads splits 65-128)"),
    (3, 6, 3, 48, 20, 64, 1, 1, "D = 48 (not a multiple of 64), group 2"),
    (2, 8, 8, 16, 5, 8, 1, 1, "no grouping (H = KV), past + M = max_t"),
    (1, 14, 2, 64, 1000, 1024, 1, 16, "0.5B heads over 1001 positions: 16 key splits"),
    (2, 4, 1, 64, 600, 1024, 1, 10, "4 heads on one kv head: 10 key splits"),
    (520, 1, 1, 16, 0, 1024, 1, 1, "520 rows from position 0: enough workgroups, one split"),
    (600, 8, 1, 64, 500, 1100, 8, 1, "8 heads on one kv head, 1100 positions: runs of 8 heads, one split"),
    (1, 8, 2, 256, 700, 1024, 1, 11, "D = 256: one head per run, 11 key splits"),
    (32, 128, 8, 256, 600, 640, 4, 1, "workspace cap: 32 rows x 128 heads of 256 leave room for one split"),
]


def _setup(ql, ctx, M, H, KV, D, past, max_t, seed):
    rng = np.random.default_rng(seed)
    T = past + M
    rows = rng.standard_normal((T, KV * D)).astype(np.float32), rng.standard_normal((T, KV * D)).astype(np.float32)
    q = rng.standard_normal((M, H, D)).astype(np.float32)
    lay = ql.ArenaLayout()
    src = [lay.take(T * KV * D * 4) for _ in range(2)]
    q_off, o_off = lay.take(q.nbytes), lay.take(q.nbytes)
    act = ctx.arena(lay.used)
    for off, r in zip(src, rows):
        act.write(off, r)
    act.write(q_off, q)
    clay = ql.ArenaLayout()
    k_off, v_off = clay.take(max_t * KV * D * 4), clay.take(max_t * KV * D * 4)
    cache = ctx.arena(clay.used)
    return rows, q, act, src, q_off, o_off, cache, k_off, v_off


@pytest.mark.parametrize("M,H,KV,D,past,max_t,hpr,nsplit,label", CASES)
def test_attention_matches_oracle(ql, ctx, orc, M, H, KV, D, past, max_t, hpr, nsplit, label):
    plan = ql.plan_attention(max_t, M, H, KV, D, past)
    say(f"attention {label}: M={M} H={H} KV={KV} D={D} past={past} max_t={max_t}: heads per run "
        f"{plan.heads_per_run}, {plan.nsplit} key splits, {plan.workgroups} workgroups")
    assert (plan.heads_per_run, plan.nsplit) == (hpr, nsplit)
    rows, q, act, src, q_off, o_off, cache, k_off, v_off = _setup(ql, ctx, M, H, KV, D, past, max_t, 0xA77 + past)
    T = past + M
    # the cache filled the way a step does it: earlier positions, then this call's rows
    for off, c_off in zip(src, (k_off, v_off)):
        if past:
            ctx.kv_store(act, off, cache, c_off, max_t, past, KV * D, 0)
        ctx.kv_store(act, off + past * KV * D * 4, cache, c_off, max_t, M, KV * D, past)
    for c_off, r in zip((k_off, v_off), rows):
        assert np.array_equal(cache.read(c_off, (T, KV * D), np.float32).view(np.uint32), r.view(np.uint32))
    ctx.attention_decode(act, q_off, cache, k_off, v_off, max_t, M, H, KV, D, past, o_off)
    got = act.read(o_off, (M, H, D), np.float32)
    ref = orc.attention_gqa_cache(q, rows[0], rows[1], H, KV, D, past)
    ok, ma, mr = orc.check_tolerance(got, ref, ATOL, RTOL)
    assert ok, (label, ma, mr)
    ctx.attention_decode(act, q_off, cache, k_off, v_off, max_t, M, H, KV, D, past, o_off)
    assert np.array_equal(act.read(o_off, (M, H, D), np.float32).view(np.uint32), got.view(np.uint32))
    act.release()
    cache.release()


def test_attention_and_store_errors(ql, ctx):
    M, H, KV, D, past, max_t = 2, 4, 2, 16, 6, 8
    rows, q, act, src, q_off, o_off, cache, k_off, v_off = _setup(ql, ctx, M, H, KV, D, past, max_t, 1)
    with pytest.raises(ql.QlError):          # past + M > max_t (qwen.ts:352-355)
        ctx.attention_decode(act, q_off, cache, k_off, v_off, max_t, M, H, KV, D, past + 1, o_off)
    with pytest.raises(ql.QlError):
        ctx.kv_store(act, src[0], cache, k_off, max_t, 3, KV * D, 6)
    with pytest.raises(ql.QlError):          # H not a multiple of KV
        ctx.attention_decode(act, q_off, cache, k_off, v_off, max_t, M, 3, KV, D, past, o_off)
    with pytest.raises(ql.QlError):          # q and out overlap
        ctx.attention_decode(act, q_off, cache, k_off, v_off, max_t, M, H, KV, D, past, q_off)
    act.release()
    cache.release()


def test_kv_cache_decode_steps(ql, ctx, orc):
    """The host mirror's cache over a few decode steps of a 2-layer 0.5B-shaped config: store this
    step's k/v row at position t, attend over 0 .. t; every step matches the oracle."""
    cfg = gptq.QwenConfig(vocab_size=512, block_size=32, n_layer=2, n_head=14, n_kv_head=2, n_embd=896,
                          intermediate=640)
    kv = gptq.KvCache(ctx, cfg)
    pool = gptq.ActivationArena(ctx, 1 << 20)
    D, R = kv.D, kv.row_len
    rng = np.random.default_rng(3)
    hist = {l: ([], []) for l in range(cfg.n_layer)}
    for t in range(5):
        for layer in range(cfg.n_layer):
            k, v = (rng.standard_normal((1, R)).astype(np.float32) for _ in range(2))
            q = rng.standard_normal((1, cfg.n_head * D)).astype(np.float32)
            K, V, Q, O = pool.alloc((1, R)), pool.alloc((1, R)), pool.alloc((1, cfg.n_head * D)), pool.alloc((1, cfg.n_head * D))
            K.write(k)
            V.write(v)
            Q.write(q)
            kv.store(layer, K, V, 1, t)
            kv.attend(layer, Q, O, 1, t)
            hist[layer][0].append(k)
            hist[layer][1].append(v)
            ref = orc.attention_gqa_cache(q.reshape(1, cfg.n_head, D), np.concatenate(hist[layer][0]),
                                          np.concatenate(hist[layer][1]), cfg.n_head, cfg.n_kv_head, D, t)
            ok, ma, _ = orc.check_tolerance(O.read(), ref, ATOL, RTOL)
            assert ok, (t, layer, ma)
            pool.reset()
    with pytest.raises(ql.QlError):
        Q, O = pool.alloc((1, cfg.n_head * D)), pool.alloc((1, cfg.n_head * D))
        kv.attend(0, Q, O, 1, cfg.block_size)
    kv.release()
