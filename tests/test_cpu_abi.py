"""CPU: libferrum_kv.so loads and exports every entry point include/ferrum_kv.h
declares; argument validation that happens before any device work returns the
reference's error variants and strings (no kernel is launched here)."""
import ctypes
import os
import re
import struct

import pytest

import ferrum_amd as fa
from ferrum_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    names = []
    for h in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if h.endswith(".h"):
            text = open(os.path.join(ROOT, "include", h)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names += re.findall(r"^\s*[A-Za-z_][\w\s\*]*?\b(fkv_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_every_declared_entry_point_is_exported_and_bound():
    names = header_functions()
    assert len(names) >= 30
    lib = _lib.load()
    for n in names:
        assert hasattr(lib, n), f"{n} declared but not exported"
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert sorted(_lib.SIGNATURES) == names


def test_abi_version_and_device_count():
    lib = _lib.load()
    assert lib.fkv_abi_version() == 2 == _lib.ABI_VERSION
    assert lib.fkv_device_count() >= 0


def _create(**kw):
    base = dict(n_layers=2, n_kv_heads=2, head_dim=64, num_blocks=4)
    base.update(kw)
    return fa.PagedKvPool(fa.PagedConfig(**base))


@pytest.mark.parametrize("field", ["n_layers", "n_kv_heads", "head_dim", "num_blocks", "block_size"])
def test_zero_dimension_is_cache_error(field):
    # pool.rs:28 "kv pool dimension is zero", checked before any allocation
    with pytest.raises(fa.CacheError, match="^cache: kv pool dimension is zero$"):
        _create(**{field: 0})


def test_config_validation_messages():
    with pytest.raises(fa.KernelError, match="^kernel: q8_0 k is not a multiple of 32$"):
        _create(kv_dtype=fa.DTYPE_Q8_0, head_dim=48)
    # the Q8_0 tile order works in 16-token sub-tiles of 64-dim operand runs
    for bad in ({"head_dim": 96}, {"block_size": 8}):
        with pytest.raises(fa.KernelError, match="^kernel: q8_0 kv needs head_dim % 64 == 0"):
            _create(kv_dtype=fa.DTYPE_Q8_0, **bad)
    with pytest.raises(fa.KernelError, match="^kernel: unsupported dtype$"):
        _create(kv_dtype=3)
    with pytest.raises(fa.InvalidRequest, match="unknown f16 rounding mode"):
        _create(f16_rounding=7)
    with pytest.raises(fa.CacheError, match="^cache: kv pool size overflow$"):
        _create(num_blocks=1 << 40)
    with pytest.raises(fa.CacheError, match="^cache: kv pool dimension is zero$"):
        fa.PreallocatedKvPool.new(fa.KvPoolConfig(0, 1, 4, 3, 2))
    with pytest.raises(fa.CacheError, match="^cache: kv pool size overflow$"):
        fa.PreallocatedKvPool.new(fa.KvPoolConfig(1 << 20, 1 << 20, 1 << 20, 1 << 20, 2))


def test_null_arguments_are_invalid_request():
    lib = _lib.load()
    assert lib.fkv_paged_create(None, None) == _lib.FKV_ERR_INVALID
    assert lib.fkv_last_error() == b"null argument"
    assert lib.fkv_append(None, 0, None, None, None, 0, None) == _lib.FKV_ERR_INVALID
    assert lib.fkv_device_copy(ctypes.c_void_p(16), ctypes.c_void_p(8), 16, None) == _lib.FKV_ERR_INVALID
    assert b"16-byte aligned" in lib.fkv_last_error()


def test_destroy_and_close_keep_the_last_error(tmp_path):
    # finalizers may run between a failing call and the read of its message
    lib = _lib.load()
    assert lib.fkv_paged_create(None, None) == _lib.FKV_ERR_INVALID
    for destroy in (lib.fkv_paged_destroy, lib.fkv_kvpool_destroy, lib.fkv_seqs_destroy,
                    lib.fkv_gguf_close):
        assert destroy(None) == _lib.FKV_OK
        assert lib.fkv_last_error() == b"null argument"
    good = tmp_path / "ok.gguf"
    good.write_bytes(b"GGUF" + struct.pack("<IQQ", 3, 0, 0) + bytes(8))  # data at 32
    f = fa.GgufFile(str(good))
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGUF" + struct.pack("<I", 3))
    assert lib.fkv_gguf_open(str(bad).encode(), ctypes.byref(ctypes.c_void_p())) == _lib.FKV_ERR_GGUF
    f.close()
    assert lib.fkv_last_error().startswith(b"gguf: ")
    # any other successful call clears the thread's message
    fa.GgufFile(str(good)).close()
    assert lib.fkv_last_error() == b""


def test_error_classes_mirror_ferrum_error():
    # FerrumError Display (core-types/src/error.rs:21-46) and HTTP mapping (:101)
    assert fa.Unavailable("no free kv blocks").http_status == 503
    assert fa.InvalidRequest("x").http_status == 400
    assert issubclass(fa.CacheError, fa.FerrumError)


def test_static_scratch_size_matches_the_header():
    text = open(os.path.join(ROOT, "include", "ferrum_kv.h")).read()
    m = re.search(r"#define FKV_STATIC_SCRATCH_BYTES \((\d+)ull << (\d+)\)", text)
    assert m, "FKV_STATIC_SCRATCH_BYTES missing from ferrum_kv.h"
    assert int(m.group(1)) << int(m.group(2)) == _lib.STATIC_SCRATCH_BYTES


def test_set_tuning_checks_its_arguments():
    lib = _lib.load()
    assert lib.fkv_set_tuning(99, 0) == _lib.FKV_ERR_INVALID
    assert lib.fkv_set_tuning(_lib.TUNE_ATTN_SPLIT_TOKENS, 24) == _lib.FKV_ERR_INVALID
    assert lib.fkv_set_tuning(_lib.TUNE_ATTN_ORDER, 3) == _lib.FKV_ERR_INVALID
    assert lib.fkv_set_tuning(_lib.TUNE_ATTN_STREAM, 2) == _lib.FKV_ERR_INVALID
    assert lib.fkv_set_tuning(_lib.TUNE_PREFILL_SPLIT_BLOCKS, -2) == _lib.FKV_ERR_INVALID
    assert lib.fkv_set_tuning(_lib.TUNE_ATTN_ENGINE, 2) == _lib.FKV_ERR_INVALID
    assert lib.fkv_set_tuning(_lib.TUNE_ATTN_WGS_PER_CU, 1) == _lib.FKV_ERR_INVALID
    assert lib.fkv_set_tuning(_lib.TUNE_ATTN_WGS_PER_CU, 4) == _lib.FKV_ERR_INVALID
    for knob, value, default in ((_lib.TUNE_ATTN_SPLIT_TOKENS, 512, 0),
                                 (_lib.TUNE_ATTN_ORDER, 1, -1),
                                 (_lib.TUNE_ATTN_STREAM, 1, 0),
                                 (_lib.TUNE_PREFILL_SPLIT_BLOCKS, 7, -1),
                                 (_lib.TUNE_ATTN_ENGINE, 1, 0),
                                 (_lib.TUNE_ATTN_WGS_PER_CU, 2, 0)):
        assert lib.fkv_set_tuning(knob, value) == _lib.FKV_OK
        assert lib.fkv_set_tuning(knob, default) == _lib.FKV_OK


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    """Without the built library every product call raises; nothing falls back to the CPU."""
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "libferrum_kv.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(RuntimeError, match="is missing: .*no CPU fallback"):
        _lib.load()
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        fa.PagedKvPool(fa.PagedConfig(n_layers=1, n_kv_heads=2, head_dim=64, num_blocks=16))
