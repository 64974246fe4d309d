"""zk_cache_write_batch_qkv on the MI355X: the fused q/k/v projection and
KV write of a runner step against the two-call sequence it replaces (the
projection, then zk_cache_write_batch of its K and V columns) through the
projection configuration the call ran (zk_linear_choice: the weight-streaming
kernel with split k whose sums the write kernel adds, or zk_linear's own
choice).  Two caches with the same history, one written each way: the q
columns and every pool byte must agree bit for bit.  Covered: a decode step
of 48 sequences with forks whose first write copies a shared tail block
(T <= 64: the folded form when the plan keeps a split), a prefill step of
T > 64 (the projection, then the append), bf16 and fp8 pools (fp8 always
takes the two-step form, quantising in the append), and the bf16 decode
step with its plan pinned to a split of k (zk_linear_pin_split), so the
folded kernel is covered whatever the tuning keeps."""
import numpy as np
import pytest
import torch

import oracle
from tests.gpu_util import announce, normal, to_dev

pytestmark = pytest.mark.gpu

H, HKV, D, BS, HID = 32, 8, 128, 16, 4096
COLS = (H + 2 * HKV) * D


def _twins(kv, layers, seqs, rng):
    """Two caches with identical blocks and contents: seqs {id: tokens}."""
    import zealot_amd as ze
    from zealot_amd import KVCache
    cdt = {"bf16": torch.bfloat16, "fp8": torch.float8_e4m3fn}[kv]
    nb = sum((t + 40) // BS + 2 for t in seqs.values()) + 64
    out = []
    for _ in range(2):
        bm = ze.BlockManager(nb, BS)
        out.append((KVCache(nb, BS, layers, HKV, D, dtype=cdt, max_seqs=96, max_blocks_per_seq=16), bm))
    init = {s: [to_dev(normal(rng, (t, HKV, D), oracle.BF16)) for _ in range(2 * layers)] for s, t in seqs.items()}
    for cache, bm in out:
        for s, t in seqs.items():
            cache.register_seq(s, 16)
            for _ in range((t + 40) // BS + 1):
                cache.alloc_block(s, bm)
            if kv == "fp8":
                cache.set_fp8_scales(s, np.full((layers, HKV), 0.05, np.float32), np.full((layers, HKV), 0.04, np.float32))
            for layer in range(layers):
                cache.write_batch(layer, [s], [t], init[s][2 * layer], init[s][2 * layer + 1])
    return out


def _reference(x, w, kv):
    """The projection through the configuration zk_cache_write_batch_qkv ran."""
    from zealot_amd import dense
    ch = dense.linear_choice(x.shape[0], COLS, HID)
    if kv == "bf16" and ch["fused_splits"] > 1:
        return dense.linear_skinny(x, w, ch["fused_splits"], ch["fused_rows"]), ch
    return dense.linear(x, w), ch


def _same(a, b):
    return torch.equal(a.contiguous().view(torch.uint8), b.contiguous().view(torch.uint8))


@pytest.mark.parametrize("kv,pin", [("bf16", 0), ("fp8", 0), ("bf16", 4)])
def test_write_batch_qkv_is_projection_then_write_bit_for_bit(kv, pin):
    """pin > 1: the decode step's plan is pinned to that split of k over
    64-row tiles, so the folded reduce + KV write kernel runs whatever the
    tuning chose."""
    from zealot_amd import dense
    rng = np.random.default_rng({"bf16": 71, "fp8": 72}[kv] + pin)
    layers = 2
    base = {f"s{i}": int(rng.integers(1, 40)) for i in range(44)}
    base["par"] = 2 * BS + 5  # forked below: its children's first write copies the partial tail block
    (ca, bma), (cb, bmb) = _twins(kv, layers, base, rng)
    kids = ["k0", "k1", "k2", "k3"]
    for cache in (ca, cb):
        for k in kids:
            cache.fork_seq("par", k)
    w = to_dev((oracle.bf16_bits_from_f32((rng.standard_normal((COLS, HID)) / np.sqrt(HID)).astype(np.float32)))
               .reshape(COLS, HID))
    steps = [([s for s in base if s != "par"] + kids, None),                 # decode: 48 rows
             (["s0", "s1", "s2"], [40, 40, 40])]                             # prefill: 120 rows
    if pin:
        dense.linear(to_dev(normal(rng, (48, HID), oracle.BF16)), w)  # makes the decode step's plan
        dense.pin_split(48, COLS, HID, pin, 64)
    for ids, nt in steps:
        nt = nt or [1] * len(ids)
        T = sum(nt)
        for layer in range(layers):
            announce(f"write_batch_qkv {kv} T={T} layer={layer}")
            x = to_dev(normal(rng, (T, HID), oracle.BF16))
            qkv = ca.write_batch_qkv(layer, ids, nt, x, w, H)
            y, ch = _reference(x, w, kv)
            cb.write_batch(layer, ids, nt, y[:, H * D:(H + HKV) * D].view(T, HKV, D), y[:, (H + HKV) * D:].view(T, HKV, D))
            torch.cuda.synchronize()
            if pin and T <= 64:
                assert ch["fused_splits"] == pin, ch  # the folded kernel ran
            assert _same(qkv[:, :H * D], y[:, :H * D]), ch
            for pa, pb in ((ca.k_pool(layer), cb.k_pool(layer)), (ca.v_pool(layer), cb.v_pool(layer))):
                assert _same(pa, pb), (ch, layer, T)
    par = ca.seq_state("par").block_ids
    for k in kids:  # the forks' partial tails were copied, the full blocks before them stay shared
        ids_k = ca.seq_state(k).block_ids
        assert ids_k[2] != par[2] and ids_k[:2] == par[:2]


def test_write_batch_qkv_rejects_bad_shapes():
    import zealot_amd as ze
    from zealot_amd import KVCache
    from zealot_amd._lib import ZealotError
    bm = ze.BlockManager(16, BS)
    cache = KVCache(16, BS, 1, HKV, D, dtype=torch.bfloat16, max_seqs=4, max_blocks_per_seq=4)
    cache.register_seq("a", 4)
    cache.alloc_block("a", bm)
    x = torch.zeros((1, 256), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros((COLS, 256), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        cache.write_batch_qkv(0, ["a"], [1], x, w[:, :128], H)
    with pytest.raises(TypeError):
        cache.write_batch_qkv(0, ["a"], [1], x.float(), w, H)
    with pytest.raises(ZealotError):  # no block for a 17th token
        cache.write_batch_qkv(0, ["a"], [17], torch.zeros((17, 256), dtype=torch.bfloat16, device="cuda"), w, H)
    with pytest.raises(ValueError):  # out of the wrong shape
        cache.write_batch_qkv(0, ["a"], [1], x, w, H, out=torch.empty((1, 64), dtype=torch.bfloat16, device="cuda"))
    buf = torch.zeros(COLS + 256, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ZealotError):  # out overlapping x
        cache.write_batch_qkv(0, ["a"], [1], buf[:256].view(1, 256), w, H, out=buf[128:128 + COLS].view(1, COLS))
    assert cache.seq_state("a").cached_tokens == 0  # nothing was written
