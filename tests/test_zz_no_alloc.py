"""zk_paged_decode_noalloc against zk_paged_decode, both called through the C
ABI on the same inputs: two calls in a row, the second with a smaller batch
(the scratch keeps the first call's contents), for the MFMA bf16 path, the
fp8 path and the generic fp32 path.  The two entry points run the same
kernels with the same work split, so their outputs must be identical; the
second call is also checked against the CPU oracle (2e-2 bf16, 1e-5 fp32)."""
import ctypes
import math

import numpy as np
import pytest
import torch

import oracle
from tests.gpu_util import announce, as_f32, decode_case, max_abs_err, to_dev, to_host
from zealot_amd import _lib

pytestmark = pytest.mark.gpu

SCRATCH = 64 << 20


def _call(noalloc, q, kp, vp, bt, lens, ks=None, vs=None):
    L = _lib.lib()
    n, h, d = q.shape
    nb, hkv, bs, _ = kp.shape
    out = torch.full_like(q, float("nan"))
    qdt = _lib.F32 if q.dtype == torch.float32 else _lib.BF16
    kvdt = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.uint8: _lib.FP8_E4M3}[kp.dtype]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = (q.data_ptr(), qdt, kp.data_ptr(), vp.data_ptr(), kvdt, out.data_ptr(), bt.data_ptr(), lens.data_ptr(),
            n, h, hkv, d, bs, bt.shape[1], nb, 1.0 / math.sqrt(d), _lib.GQA_GROUPED,
            ks.data_ptr() if ks is not None else None, vs.data_ptr() if vs is not None else None)
    if noalloc:
        rc = L.zk_paged_decode_noalloc(*args, stream)
    else:
        need = L.zk_paged_decode_workspace_size(n, h, d, bt.shape[1], bs)
        ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        rc = L.zk_paged_decode(*args, ws.data_ptr(), need, stream)
    assert rc == 0, L.zk_last_error().decode()
    torch.cuda.synchronize()
    return out


def _case(seed, H, Hkv, D, lens, dt):
    q, kp, vp, bt, nb = decode_case(seed, H, Hkv, D, lens, dt)
    return (q, kp, vp, bt, lens), (to_dev(q), to_dev(kp), to_dev(vp), to_dev(bt),
                                   to_dev(np.asarray(lens, np.int32)))


def _oracle(host, dt):
    q, kp, vp, bt, lens = host
    return oracle.paged_decode(as_f32(q, dt), kp, vp, dt, bt, lens, kp.shape[1], kp.shape[3], kp.shape[2],
                               np.float32(1.0 / math.sqrt(kp.shape[3])), oracle.GROUPED, threads=8)


@pytest.mark.parametrize("H,Hkv,D,dt,tol", [
    (32, 8, 128, oracle.BF16, 2e-2),   # C2 heads: MFMA kernel, split partitions + reduce
    (4, 4, 32, oracle.F32, 1e-5),      # C1 heads: generic kernel
])
def test_noalloc_matches_workspace_entry_point(H, Hkv, D, dt, tol):
    rng = np.random.default_rng(31 + D)
    big = [int(x) for x in rng.integers(1, 6000, 48)] + [8192, 1, 0]
    small = [5, 700, 16, 3000, 33]
    for i, lens in enumerate((big, small)):
        announce(f"noalloc decode H{H}/Hkv{Hkv}/D{D} dt={dt} call {i} N={len(lens)}")
        host, dev = _case(40 + i, H, Hkv, D, lens, dt)
        a = _call(True, *dev)
        b = _call(False, *dev)
        assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a,
                           b.view(torch.int16) if b.dtype == torch.bfloat16 else b)
        got = as_f32(to_host(a), dt)
        assert max_abs_err(got, _oracle(host, dt)) <= tol


def test_noalloc_fp8_two_calls():
    from zealot_amd import ops
    H, Hkv, D, BS = 32, 8, 128, 16
    for i, lens in enumerate(([1024, 5000, 2048, 16384, 1100], [1500, 1024])):
        announce(f"noalloc decode fp8 call {i} lens={lens}")
        rng = np.random.default_rng(50 + i)
        from tests.gpu_util import normal, paged_tables
        bt, nb = paged_tables(rng, lens, BS)
        T = sum(lens)
        k = to_dev(normal(rng, (T, Hkv, D), oracle.BF16))
        v = to_dev(normal(rng, (T, Hkv, D), oracle.BF16))
        q = to_dev(normal(rng, (len(lens), H, D), oracle.BF16))
        cu = to_dev(np.concatenate([[0], np.cumsum(lens)]).astype(np.int64))
        slots = np.concatenate([bt[n, np.arange(L) // BS].astype(np.int64) * BS + np.arange(L) % BS
                                for n, L in enumerate(lens)])
        rows = np.repeat(np.arange(len(lens)), lens).astype(np.int32)
        ks, vs = ops.fp8_scales(k, cu), ops.fp8_scales(v, cu)
        kp = torch.zeros((nb, Hkv, BS, D), dtype=torch.uint8, device="cuda")
        vp = torch.zeros_like(kp)
        ops.append(kp, vp, k, v, to_dev(slots), k_scales=ks, v_scales=vs, token_row=to_dev(rows))
        dev = (q, kp, vp, to_dev(bt), to_dev(np.asarray(lens, np.int32)))
        a = _call(True, *dev, ks=ks, vs=vs)
        b = _call(False, *dev, ks=ks, vs=vs)
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_noalloc_rejects_oversized_call_and_launches_nothing():
    L = _lib.lib()
    # every buffer has the full shape of the call (so nothing could read out
    # of bounds even if it launched): 4096 sequences x 64 heads, tables of
    # 4096 entries (all block 0), context 1
    q = torch.zeros((4096, 64, 128), dtype=torch.float32, device="cuda")
    out = torch.full_like(q, 7.0)
    pool = torch.zeros((16, 4, 16, 128), dtype=torch.float32, device="cuda")
    bt = torch.zeros((4096, 4096), dtype=torch.int32, device="cuda")
    lens = torch.ones(4096, dtype=torch.int32, device="cuda")
    # 4096 sequences' worth of fp32 partitions does not fit: the host check fails
    rc = L.zk_paged_decode_noalloc(q.data_ptr(), _lib.F32, pool.data_ptr(), pool.data_ptr(), _lib.F32,
                                   out.data_ptr(), bt.data_ptr(), lens.data_ptr(), 4096, 64, 4, 128, 16, 4096, 16,
                                   0.1, _lib.GQA_GROUPED, None, None, None)
    assert rc == _lib.ERR_INVALID_ARGUMENT
    assert "bytes of scratch, the maximum is 67108864" in L.zk_last_error().decode()
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())


_MEM_PROBE = r"""
import ctypes, json, math, sys
import torch
sys.path.insert(0, sys.argv[1])
from zealot_amd import _lib

L = _lib.lib()
dev = "cuda"
N, H, Hkv, D, BS, NB, MB = 8, 32, 8, 128, 16, 64, 8
kp = torch.zeros((NB, Hkv, BS, D), dtype=torch.bfloat16, device=dev)
vp = torch.zeros_like(kp)
k = torch.randn((N * MB * BS, Hkv, D), device=dev).to(torch.bfloat16)
v = torch.randn_like(k)
slots = torch.arange(N * MB * BS, dtype=torch.int64, device=dev)
q = torch.randn((N, H, D), device=dev).to(torch.bfloat16)
out = torch.empty_like(q)
bt = torch.arange(N * MB, dtype=torch.int32, device=dev).view(N, MB)
lens = torch.full((N,), MB * BS, dtype=torch.int32, device=dev)
need = L.zk_paged_decode_workspace_size(N, H, D, MB, BS)
ws = torch.empty(need, dtype=torch.uint8, device=dev)
s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
torch.cuda.synchronize()

def free():
    torch.cuda.synchronize()
    return torch.cuda.mem_get_info()[0]

f = [free()]
assert L.zk_append(kp.data_ptr(), vp.data_ptr(), _lib.BF16, k.data_ptr(), v.data_ptr(), _lib.BF16,
                   slots.data_ptr(), k.shape[0], Hkv, D, BS, NB, None, None, None, s) == 0
f.append(free())
args = (q.data_ptr(), _lib.BF16, kp.data_ptr(), vp.data_ptr(), _lib.BF16, out.data_ptr(), bt.data_ptr(),
        lens.data_ptr(), N, H, Hkv, D, BS, MB, NB, 1.0 / math.sqrt(D), _lib.GQA_GROUPED, None, None)
assert L.zk_paged_decode(*args, ws.data_ptr(), need, s) == 0
f.append(free())
assert L.zk_paged_decode_noalloc(*args, s) == 0
f.append(free())
assert L.zk_paged_decode_noalloc(*args, s) == 0
f.append(free())
print(json.dumps(f))
"""


def test_noalloc_scratch_reserved_by_its_first_call():
    """The 64 MiB scratch is reserved on a GPU by the first
    zk_paged_decode_noalloc call there, not by the library's other kernels:
    device memory free (hipMemGetInfo) in a fresh process before and after the
    first zk_append, the first zk_paged_decode and two no-alloc calls."""
    import json
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    announce("noalloc scratch reservation probe (fresh process)")
    r = subprocess.run([sys.executable, "-c", _MEM_PROBE, root], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    f = json.loads(r.stdout.strip().splitlines()[-1])
    mib = [(a - b) / 2**20 for a, b in zip(f, f[1:])]
    print(f"[gpu-case] MiB reserved by: first append {mib[0]:.1f}, first decode {mib[1]:.1f}, "
          f"first no-alloc decode {mib[2]:.1f}, second {mib[3]:.1f}", flush=True)
    assert mib[0] < 32 and mib[1] < 32, mib    # code objects only, no scratch
    assert mib[2] >= SCRATCH / 2**20, mib      # the scratch arrives with the first no-alloc call
    assert abs(mib[3]) < 1, mib                # and is not reserved again


def test_noalloc_under_graph_capture():
    """One eager call (looks the scratch up), then zk_paged_decode_noalloc
    captured in a HIP graph through torch.cuda.graph and replayed on new q
    values, eager work and synchronisation between the replays: every replay
    bit for bit equal to the workspace entry point on the same q."""
    H, Hkv, D = 32, 8, 128
    rng = np.random.default_rng(77)
    lens = [int(x) for x in rng.integers(1, 5000, 40)] + [8192, 1]
    host, (q, kp, vp, bt, ln) = _case(70, H, Hkv, D, lens, oracle.BF16)
    announce(f"noalloc decode under graph capture N={len(lens)}")
    L = _lib.lib()
    n = len(lens)
    out = torch.empty_like(q)
    _call(True, q, kp, vp, bt, ln)  # eager first call on this device
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        rc = L.zk_paged_decode_noalloc(q.data_ptr(), _lib.BF16, kp.data_ptr(), vp.data_ptr(), _lib.BF16,
                                       out.data_ptr(), bt.data_ptr(), ln.data_ptr(), n, H, Hkv, D, 16, bt.shape[1],
                                       kp.shape[0], 1.0 / math.sqrt(D), _lib.GQA_GROUPED, None, None, s)
    assert rc == 0, L.zk_last_error().decode()
    g = torch.Generator(device="cuda").manual_seed(78)
    for rep in range(4):
        q.copy_(torch.randn(q.shape, generator=g, device="cuda").to(torch.bfloat16))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = _call(False, q, kp, vp, bt, ln)
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), rep
        _call(True, q, kp, vp, bt, ln)  # eager work on the same scratch between replays
