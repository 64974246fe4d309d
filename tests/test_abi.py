"""The C ABI library: loads, exports every symbol include/*.h declares,
and rejects bad arguments on the host before any GPU work (no compute calls
here, so these run without a GPU)."""
import ctypes
import glob
import os
import re
import subprocess

import pytest

import zealot_amd
from zealot_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "zealot_kv.h")
HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))


def declared_functions():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"\b(zk_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_header_declares_the_boundary():
    names = declared_functions()
    for must in ("zk_append", "zk_gather", "zk_copy_blocks", "zk_paged_decode", "zk_bm_allocate",
                 "zk_cache_store_kv", "zk_cache_append_kv", "zk_last_error"):
        assert must in names


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    missing = [n for n in declared_functions() if not hasattr(L, n)]
    assert not missing, missing
    # the ctypes table covers the header exactly
    assert sorted(_lib.SIGNATURES) == declared_functions()


def test_exports_with_nm():
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (zk_[a-z0-9_]+)\b", out))
    assert set(declared_functions()) <= exported


@pytest.mark.parametrize("header", ["zealot_kv.h", "zealot_sched.h", "zealot_dense.h"])
def test_header_compiles_as_c(header):
    src = f'#include "{header}"\nint main(void){{return ZK_OK;}}\n'
    r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-fsyntax-only",
                        "-I", os.path.dirname(HEADER), "-x", "c", "-"], input=src,
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_abi_version():
    assert _lib.lib().zk_abi_version() == 1


def _err(rc):
    return rc, _lib.lib().zk_last_error().decode()


def test_append_rejects_bad_arguments_on_host():
    L = _lib.lib()
    dummy = ctypes.c_void_p(0x1000)
    rc, msg = _err(L.zk_append(dummy, dummy, 7, dummy, dummy, _lib.BF16, dummy, 4, 8, 128, 16, 10,
                               None, None, None, None))
    assert rc == _lib.ERR_INVALID_ARGUMENT and "dtype" in msg
    rc, msg = _err(L.zk_append(dummy, dummy, _lib.FP8_E4M3, dummy, dummy, _lib.BF16, dummy, 4, 8,
                               128, 16, 10, None, None, None, None))
    assert rc == _lib.ERR_INVALID_ARGUMENT and "scales" in msg
    rc, msg = _err(L.zk_append(dummy, dummy, _lib.BF16, dummy, dummy, _lib.BF16, dummy, 4, 0, 128,
                               16, 10, None, None, None, None))
    assert rc == _lib.ERR_INVALID_ARGUMENT
    # zero tokens is a no-op
    assert L.zk_append(None, None, _lib.BF16, None, None, _lib.BF16, None, 0, 8, 128, 16, 10,
                       None, None, None, None) == _lib.OK


def test_linear_skinny_rejects_bad_shapes_on_host():
    """The weight-streaming GEMM's limits are checked before any device call."""
    L = _lib.lib()
    d = ctypes.c_void_p(0x1000)
    bad = [
        (65, 4096, 4096, _lib.BF16, 128, 1),    # m > 64
        (8, 4096 + 64, 4096, _lib.BF16, 128, 1),  # n not a multiple of the tile rows
        (8, 4096, 4096 + 64, _lib.BF16, 64, 1),   # k not a multiple of 128 * splits
        (8, 4096, 4096, _lib.BF16, 64, 64),     # k % (128 * splits) != 0
        (8, 4096, 4096, _lib.BF16, 96, 1),      # tile rows neither 64 nor 128
        (64, 524288, 4096, _lib.BF16, 128, 2),  # split sums beyond the 32 MiB workspace
        (8, 4096, 4096, _lib.FP8_E4M3, 128, 1),  # output dtype
    ]
    for m, n, k, od, rows, splits in bad:
        rc, msg = _err(L.zk_linear_skinny(d, d, d, m, n, k, od, rows, splits, None))
        assert rc == _lib.ERR_INVALID_ARGUMENT, (m, n, k, rows, splits, msg)
        assert "zk_linear_skinny" in msg


def test_decode_rejects_bad_arguments_on_host():
    L = _lib.lib()
    d = ctypes.c_void_p(0x1000)
    base = dict(q=d, qd=_lib.BF16, k=d, v=d, kvd=_lib.BF16, o=d, bt=d, sl=d, n=4, h=32, hkv=8,
                dim=128, bs=16, mb=16, nb=100, scale=0.1, mp=_lib.GQA_GROUPED, ks=None, vs=None,
                ws=d, wsb=1 << 30, s=None)

    def call(**kw):
        a = dict(base, **kw)
        return _err(L.zk_paged_decode(a["q"], a["qd"], a["k"], a["v"], a["kvd"], a["o"], a["bt"],
                                      a["sl"], a["n"], a["h"], a["hkv"], a["dim"], a["bs"], a["mb"],
                                      a["nb"], a["scale"], a["mp"], a["ks"], a["vs"], a["ws"],
                                      a["wsb"], a["s"]))

    assert call(h=30)[0] == _lib.ERR_INVALID_ARGUMENT  # 30 % 8 != 0
    assert call(dim=512)[0] == _lib.ERR_INVALID_ARGUMENT
    assert call(kvd=_lib.FP8_E4M3)[0] == _lib.ERR_INVALID_ARGUMENT  # fp8 without scales
    assert call(ks=d, vs=d)[0] == _lib.ERR_INVALID_ARGUMENT  # scales on a bf16 pool
    assert call(wsb=16)[0] == _lib.ERR_INVALID_ARGUMENT
    rc, msg = call(ws=ctypes.c_void_p(0x1001))
    assert rc == _lib.ERR_INVALID_ARGUMENT and "aligned" in msg
    assert call(mp=5)[0] == _lib.ERR_INVALID_ARGUMENT
    assert call(n=0)[0] == _lib.OK


def test_workspace_size_grows_with_context():
    L = _lib.lib()
    a = L.zk_paged_decode_workspace_size(256, 32, 128, 512, 16)
    b = L.zk_paged_decode_workspace_size(256, 32, 128, 1024, 16)
    assert 0 < a < b


def test_copy_blocks_and_gather_validate_on_host():
    L = _lib.lib()
    d = ctypes.c_void_p(0x1000)
    arr = (ctypes.c_void_p * 1)(None)
    rc, _ = _err(L.zk_copy_blocks(arr, 1, 4096, 10, d, d, 3, None))
    assert rc == _lib.ERR_INVALID_ARGUMENT  # NULL pool
    assert L.zk_copy_blocks(arr, 1, 4096, 10, d, d, 0, None) == _lib.OK
    rc, _ = _err(L.zk_gather(d, d, 9, d, 4, d, d, 1, d, d, 8, 128, 16, 10, None))
    assert rc == _lib.ERR_INVALID_ARGUMENT


def test_product_does_not_import_the_oracle():
    """The product package must never route through the CPU oracle."""
    pkg = os.path.join(ROOT, "zealot_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                assert "import oracle" not in text and "from oracle" not in text, f
                assert "zk_oracle" not in text and "liboracle" not in text, f


def test_package_imports_without_gpu():
    from zealot_amd import HipAttention, KVCache, ops  # noqa: F401
    assert callable(ops.paged_decode) and callable(ops.append)


def test_noalloc_decode_rejects_oversized_call_on_host():
    """zk_paged_decode_noalloc checks the scratch it needs before touching a
    device: 4096 sequences x 64 heads of fp32 partitions (the generic path
    cuts 4096-page tables into 256 partitions) need far more than 64 MiB."""
    L = _lib.lib()
    dummy = ctypes.c_void_p(0x1000)
    rc, msg = _err(L.zk_paged_decode_noalloc(dummy, _lib.F32, dummy, dummy, _lib.F32, dummy, dummy, dummy,
                                             4096, 64, 4, 128, 16, 4096, 16, 0.1, _lib.GQA_GROUPED, None, None,
                                             None))
    assert rc == _lib.ERR_INVALID_ARGUMENT
    assert "bytes of scratch, the maximum is 67108864" in msg
    rc, msg = _err(L.zk_paged_decode_noalloc(dummy, _lib.F32, dummy, dummy, _lib.F32, dummy, dummy, dummy,
                                             4, 30, 4, 128, 16, 64, 16, 0.1, _lib.GQA_GROUPED, None, None, None))
    assert rc == _lib.ERR_INVALID_ARGUMENT and "multiple" in msg  # argument checks come first
    assert L.zk_paged_decode_noalloc(None, _lib.F32, None, None, _lib.F32, None, None, None, 0, 4, 4, 128, 16,
                                     64, 16, 0.1, _lib.GQA_GROUPED, None, None, None) == 0  # empty batch
