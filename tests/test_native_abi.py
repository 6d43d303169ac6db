"""The C-ABI library loads in-process and exports every symbol the header declares."""

import re
from pathlib import Path

import pytest
import torch

from seqattn import _native
from seqattn.streaming import resolve_backend

HEADER = Path(__file__).resolve().parents[1] / "include" / "seqattn_hip.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int32_t|void\*|const char\*)\s+(sa_\w+)\s*\(", text, re.M)))


def test_header_and_binding_agree():
    declared = declared_functions()
    assert declared, "no declarations parsed"
    assert set(declared) == set(_native.SIGNATURES)


@pytest.mark.skipif(not _native.library_is_built(), reason="native library not built")
def test_library_loads_and_exports_every_declared_symbol():
    lib = _native.lib()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.sa_abi_version() == _native.ABI_VERSION
    assert lib.sa_last_error() == b""


@pytest.mark.skipif(not _native.library_is_built(), reason="native library not built")
def test_library_shares_torchs_hip_runtime():
    _native.lib()
    maps = Path("/proc/self/maps").read_text()
    runtimes = {line.split()[-1] for line in maps.splitlines() if "libamdhip64" in line}
    assert len(runtimes) == 1, runtimes
    assert any("libseqattn_hip.so" in line for line in maps.splitlines())


@pytest.mark.skipif(not _native.library_is_built(), reason="native library not built")
def test_argument_errors_surface_without_a_gpu():
    lib = _native.lib()
    status = lib.sa_update_attention_state(
        None, None, None, None, None, None, *([0] * 10), 4, 4, 4, 4, 12, 0, 0, 0, 1.0, 0, 0, None)
    assert status == -3  # SA_ERR_UNSUPPORTED_HEAD_DIM (12 is not a multiple of 8)
    assert b"head_dim" in lib.sa_last_error()
    status = lib.sa_update_attention_state(
        None, None, None, None, None, None, *([0] * 10), 4, 4, 4, 4, 64, 0, 0, 0, 1.0, 0, 7, None)
    assert status == -2
    with pytest.raises(RuntimeError, match="head_dim"):
        _native.check(lib.sa_finalize_attention(
            None, None, None, None, None, *([0] * 8), 4, 4, 12, 0, None), "finalize")


@pytest.mark.skipif(not _native.library_is_built(), reason="native library not built")
def test_resident_scratch_attach_rejects_bad_arguments_without_a_gpu():
    lib = _native.lib()
    assert lib.sa_pipeline_attach_resident_scratch(None, None, 0) == -1
    assert b"sa_pipeline_attach_resident_scratch" in lib.sa_last_error()


@pytest.mark.skipif(not _native.library_is_built(), reason="native library not built")
def test_head_group_pipeline_rejects_bad_plans_without_a_gpu():
    import ctypes

    lib = _native.lib()
    handle = ctypes.c_void_p()
    bufs = (ctypes.c_void_p * 2)(16, 32)
    # num_sets 3 (at most 2), then a group of 5 K/V heads out of 4, then a
    # misaligned buffer: rejected before any HIP call.
    for sets, group, q_buf in ((3, 1, bufs), (1, 5, bufs), (1, 1, (ctypes.c_void_p * 2)(17, 32))):
        status = lib.sa_pipeline_create_head_groups(ctypes.byref(handle), 0, q_buf, bufs, bufs, None, 0, sets, 64, 64,
                                                    group, 64, 8, 4, 128, 0, None, None)
        assert status == -1, (sets, group)
        assert b"sa_pipeline_create_head_groups" in lib.sa_last_error()
        assert not handle.value
    assert lib.sa_pipeline_create_head_groups(ctypes.byref(handle), 0, bufs, bufs, bufs, None, 0, 1, 64, 64, 1, 64, 8,
                                              4, 128, 9, None, None) == -2  # dtype
    assert lib.sa_pipeline_attach_host_staging(None, None, 0) == -1


def test_backend_resolution_never_falls_back_to_cpu():
    with pytest.raises(ValueError, match="not part of this package"):
        resolve_backend("reference", torch.bfloat16, torch.device("cpu"))
    with pytest.raises(ValueError, match="ROCm"):
        resolve_backend("auto", torch.bfloat16, torch.device("cpu"))
    with pytest.raises(ValueError, match="float16 or bfloat16"):
        resolve_backend("auto", torch.float32, torch.device("cuda"))
    with pytest.raises(ValueError, match="head_dim >= 16"):
        resolve_backend("triton", torch.bfloat16, torch.device("cuda"), head_dim=8)
    if not torch.cuda.is_available():
        with pytest.raises(RuntimeError, match="not available"):
            resolve_backend("hip", torch.bfloat16, torch.device("cuda"), head_dim=64)


@pytest.mark.skipif(not _native.library_is_built(), reason="native library not built")
def test_int8_update_argument_errors_surface_without_a_gpu():
    lib = _native.lib()

    def call(head_dim, dtype=0, group=64, offset=0):
        return lib.sa_update_attention_state_int8(
            *([None] * 8), *([0] * 14), 4, 4, 4, 4, head_dim, 0, 0, offset, 0, 1.0, 0, dtype, group, None)

    assert call(136) == -3 and b"multiple of 16" in lib.sa_last_error()
    assert call(256) == -3  # head_dim 256 is not covered by the INT8 path
    assert call(24) == -3
    assert call(64, dtype=5) == -2
    assert call(64, group=48) == -1 and b"power of two" in lib.sa_last_error()
    assert call(64, offset=-1) == -1
    assert call(64) == -1 and b"null pointer" in lib.sa_last_error()


@pytest.mark.skipif(not _native.library_is_built(), reason="native library not built")
def test_noalloc_entry_point_rejects_bad_arguments_before_touching_the_gpu():
    import ctypes

    lib = _native.lib()
    fake = 1 << 40  # never dereferenced: every case below is rejected by the host-side checks

    def call(cu_q, cu_k, *, heads=(8, 2), head_dim=128, dtype=0, kv_chunk=8192, q=fake, k=fake, lse=None,
             strides=None):
        qa = (ctypes.c_int64 * len(cu_q))(*cu_q)
        ka = (ctypes.c_int64 * len(cu_k))(*cu_k)
        strides = strides if strides is not None else [8 * 128] * 9
        return lib.sa_run_resident_noalloc(q, k, fake, fake, lse, *strides, qa, ka, len(cu_q) - 1,
                                           heads[0], heads[1], head_dim, dtype, kv_chunk, 0.1, 0, None)

    assert call([0, 10], [0, 10], head_dim=64) == -3 and b"head_dim 128" in lib.sa_last_error()
    assert call([0, 10], [0, 10], dtype=7) == -2
    assert call([0, 10], [0, 10], kv_chunk=100) == -1 and b"multiple of 64" in lib.sa_last_error()
    assert call([0, 10], [0, 10], q=None) == -1 and b"null" in lib.sa_last_error()
    assert call([0, 10], [0, 0]) == -1 and b"invalid bounds" in lib.sa_last_error()
    # Stride, alignment and launch-size rules of the update and transpose
    # launches are checked before the first launch is enqueued.
    for i in range(6):  # q, k, v token/head strides
        bad = [8 * 128] * 9
        bad[i] = 8 * 128 + 4
        assert call([0, 10], [0, 10], strides=bad) == -1 and b"multiples of 8" in lib.sa_last_error()
    bad = [8 * 128] * 9
    bad[2] = 1 << 24  # k token stride
    assert call([0, 10], [0, 10], strides=bad) == -1 and b"2^24" in lib.sa_last_error()
    assert call([0, 10], [0, 10], k=fake + 8) == -1 and b"16-byte aligned" in lib.sa_last_error()
    assert call([0, 10], [0, 10], lse=fake + 2) == -1 and b"16-byte aligned" in lib.sa_last_error()
    assert call([0, 1 << 30], [0, 64], heads=(64, 2)) == -1 and b"too many queries" in lib.sa_last_error()
    # 2 K/V heads x 128 x 131,072 keys x 2 bytes = 64 MiB fits; one more tile does not.
    assert call([0, 1, 2], [0, 131_072, 131_072 + 131_073]) == -1
    message = lib.sa_last_error()
    assert b"segment 1 needs" in message and b"67108864" in message


PROBE_HEADER = HEADER.parent / "seqattn_probe.h"
PROBE_LIB = Path(_native.LIB_PATH).parent / "libseqattn_probe.so"


@pytest.mark.skipif(not PROBE_LIB.exists(), reason="probe library not built")
def test_probe_library_exports_every_declared_symbol():
    import ctypes

    names = re.findall(r"^\s*(?:int32_t|int64_t|double)\s+(sa_probe_\w+)\s*\(", PROBE_HEADER.read_text(), re.M)
    assert sorted(names) == ["sa_probe_mfma", "sa_probe_mfma_flop_per_launch", "sa_probe_mfma_out_elems"]
    lib = ctypes.CDLL(str(PROBE_LIB))
    for name in names:
        assert hasattr(lib, name), name
    lib.sa_probe_mfma_out_elems.restype = ctypes.c_int64
    lib.sa_probe_mfma_flop_per_launch.restype = ctypes.c_double
    elems = lib.sa_probe_mfma_out_elems()
    assert elems == 256 * 8 * 512
    assert lib.sa_probe_mfma_flop_per_launch() == 256 * 8 * 8 * 2048 * 24 * 16 * 16 * 32 * 2
    # A null or undersized buffer is rejected before anything is enqueued.
    lib.sa_probe_mfma.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_uint32, ctypes.c_void_p]
    assert lib.sa_probe_mfma(None, elems, 1, 0, None) == -1
    assert lib.sa_probe_mfma(ctypes.c_void_p(16), elems - 1, 1, 0, None) == -1
