"""Host-side logic of paged mode: page tables, host-memory budget, the DRAM
page cache, the Q-block / K/V-fragment schedule, the aligned on-disk stores
and the INT8 storage format.  CPU only (no kernels run here).

Cases follow the reference's tests/test_paged.py, test_cache.py and
test_nvme.py where the behaviour is the same; the cache's slots are
4,096-byte record slots here (records are read into them with O_DIRECT),
so cache sizes are stated in whole 4 KiB slots.
"""

from __future__ import annotations

import errno
import itertools
import json
import math
import os

import numpy as np
import pytest
import torch

from seqattn import (
    CallbackOutputSink,
    HostMemoryPlan,
    KVLayout,
    MemoryPageSink,
    MemoryPageSource,
    NvmeOutputSink,
    NvmeQKVStore,
    NvmeQKVWriter,
    PagedAttentionConfig,
    TensorLayout,
    load_nvme_output,
)
from seqattn.cache import KVPageCache
from seqattn.nvme import DIRECT_IO_ALIGNMENT, _open_file
from seqattn.paged.runtime import validate_source_contract
from seqattn.paged.schedule import Fragment, FragmentQueue, plan_q_groups
from seqattn.paging import build_page_descriptors, pages_by_segment, replace_page
from seqattn.quantization import dequantize_int8_per_token_group, quantize_int8_per_token_group
from seqattn.storage.records import kv_record_pages, q_record_pages


def bounds(lengths):
    return torch.tensor([0, *itertools.accumulate(lengths)], dtype=torch.int32)


def small_plan(total_mib=8, pinned_mib=1, bounce_mib=2, meta_mib=1):
    return HostMemoryPlan(total_budget_bytes=total_mib * 2**20, pinned_limit_bytes=pinned_mib * 2**20,
                          bounce_limit_bytes=bounce_mib * 2**20, metadata_margin_bytes=meta_mib * 2**20)


# ----------------------------------------------------------------- page tables

def test_pages_never_cross_packed_segment_boundaries():
    q = torch.randn(53, 4, 16)
    k = torch.randn(61, 2, 16)
    cu_q, cu_k = bounds([17, 0, 36]), bounds([19, 0, 42])
    source = MemoryPageSource(q=q, k=k, v=k.clone(), cu_seqlens_q=cu_q, cu_seqlens_k=cu_k,
                              page_target_bytes=1024, block_n=16)
    for pages, b in ((source.q_pages, cu_q.tolist()), (source.kv_pages, cu_k.tolist())):
        covered = 0
        for page in pages:
            assert b[page.segment_id] <= page.token_start
            assert page.token_stop <= b[page.segment_id + 1]
            assert page.padded_tokens % 16 == 0 and page.padded_tokens >= page.valid_tokens
            covered += page.valid_tokens
        assert covered == b[-1]
        assert [p.page_id for p in pages] == list(range(len(pages)))
    assert not any(p.segment_id == 1 for p in source.q_pages + source.kv_pages)


def test_page_table_of_the_158k_token_48_head_paged_workload():
    # 256-token pages: page_target_bytes = 256 * 48 * 128 * 2 = 3 MiB, block_n 64.
    layout = KVLayout(158_208, 48, 128, "bf16", "bf16")
    pages = build_page_descriptors([0, 158_208], bytes_per_token=layout.storage_bytes_per_token,
                                   page_target_bytes=3 * 2**20, token_alignment=64)
    assert len(pages) == 618
    assert {p.valid_tokens for p in pages} == {256}
    records = kv_record_pages(pages, layout)
    assert {r.storage_bytes for r in records} == {6 * 2**20}
    assert records[-1].file_offset + records[-1].storage_bytes == 618 * 6 * 2**20


def test_record_layout_is_aligned_and_padded():
    layout = TensorLayout(37, 4, 16, "fp32")
    pages = build_page_descriptors([0, 13, 13, 37], bytes_per_token=layout.bytes_per_token,
                                   page_target_bytes=2048, token_alignment=16)
    records = q_record_pages(pages, layout)
    for rec in records:
        assert rec.file_offset % DIRECT_IO_ALIGNMENT == 0 and rec.storage_bytes % DIRECT_IO_ALIGNMENT == 0
        assert rec.payload_bytes == rec.padded_tokens * layout.bytes_per_token
        assert rec.payload_bytes + rec.padding_bytes == rec.storage_bytes
    kv = KVLayout(43, 2, 16, "bf16", "int8")
    kv_pages = build_page_descriptors([0, 17, 17, 43], bytes_per_token=kv.storage_bytes_per_token,
                                      page_target_bytes=2048, token_alignment=16)
    for rec in kv_record_pages(kv_pages, kv):
        groups = math.ceil(rec.padded_tokens / 64)
        assert rec.v_offset == rec.k_bytes == rec.padded_tokens * 2 * 16
        assert rec.scale_bytes == groups * 2 * 2
        assert rec.v_scale_offset == rec.k_scale_offset + rec.scale_bytes == 2 * rec.k_bytes + rec.scale_bytes


# ------------------------------------------------------------ host memory plan

def test_host_memory_plan_fails_immediately_on_category_overrun():
    plan = HostMemoryPlan(total_budget_bytes=8 * 2**30, pinned_limit_bytes=1 * 2**30,
                          bounce_limit_bytes=512 * 2**20, metadata_margin_bytes=128 * 2**20)
    plan.register("pinned", 1 * 2**30)
    with pytest.raises(MemoryError, match="pinned allocation"):
        plan.register("pinned", 1)
    assert plan.cache_limit_bytes == 8 * 2**30 - 1 * 2**30 - 512 * 2**20 - 128 * 2**20
    plan.register("cache", plan.cache_limit_bytes)
    with pytest.raises(MemoryError):
        plan.register("bounce", 512 * 2**20 + 1)
    snap = plan.snapshot()
    assert snap.operator_host_peak_bytes <= 8 * 2**30
    assert snap.metadata_allocated_bytes == 128 * 2**20
    with pytest.raises(RuntimeError, match="released more"):
        plan.release("bounce", 1)
    with pytest.raises(ValueError, match="unknown host allocation category"):
        plan.register("gpu", 1)


def test_host_memory_plan_rejects_reservations_without_cache_room():
    with pytest.raises(ValueError, match="no room for the DRAM cache"):
        HostMemoryPlan(total_budget_bytes=3, pinned_limit_bytes=1, bounce_limit_bytes=1, metadata_margin_bytes=1)


def test_paged_config_validation_messages():
    with pytest.raises(ValueError, match="must leave room for the DRAM cache"):
        PagedAttentionConfig(host_memory_budget_bytes=2**30, pinned_staging_budget_bytes=2**30).validate()
    with pytest.raises(ValueError, match="quant_group_tokens=64"):
        PagedAttentionConfig(quant_group_tokens=32).validate()


# ------------------------------------------------------------------ page cache

def _tiny_pages(n_tokens=80):
    layout = KVLayout(n_tokens, 1, 16, "fp32", "fp32")  # 16-token pages: 2 KiB payload, one 4 KiB record
    pages = build_page_descriptors([0, n_tokens], bytes_per_token=layout.storage_bytes_per_token,
                                   page_target_bytes=1024, token_alignment=16)
    return layout, pages


def test_two_region_cache_has_deterministic_hot_set_and_rolling_eviction():
    layout, pages = _tiny_pages()
    plan = small_plan(total_mib=2, pinned_mib=0, bounce_mib=0, meta_mib=0)
    cache = KVPageCache(pages, layout, capacity_bytes=3 * 4096, hot_fraction=2 / 3, memory_plan=plan,
                        pinned=False)
    assert cache.slot_count == 3
    assert cache.hot_page_ids == {0, 1}
    k = torch.empty((16, 1, 16))
    v = torch.empty_like(k)
    for page_id in [0, 1, 2, 3, 0, 1, 4]:
        page = pages[page_id]
        if cache.get(page, k, v).hit:
            assert torch.all(k == page_id) and torch.all(v == -page_id)
        else:
            k.fill_(page_id)
            v.fill_(-page_id)
            assert cache.put(page, k, v)
    assert cache.hits == 2 and cache.misses == 5
    # page 3 took the single rolling slot from page 2, page 4 then evicted page 3
    assert not cache.get(pages[2], k, v).hit and not cache.get(pages[3], k, v).hit
    assert cache.get(pages[4], k, v).hit and torch.all(k == 4)
    assert cache.peak_bytes <= cache.registered_bytes
    cache.close()
    assert plan.snapshot().dram_cache_allocated_bytes == 0


def test_cache_never_evicts_a_slot_with_copies_in_flight():
    layout, pages = _tiny_pages()
    cache = KVPageCache(pages, layout, capacity_bytes=2 * 4096, hot_fraction=0.0,
                        memory_plan=small_plan(), pinned=False)
    slot_a = cache.reserve(pages[0])
    cache.commit(pages[0], slot_a)
    cache.slab.hold(slot_a)                      # an H2D copy still reads it
    slot_b = cache.reserve(pages[1])
    cache.commit(pages[1], slot_b)
    assert cache.reserve(pages[2]) == slot_b     # LRU page 0 is held: page 1 is evicted instead
    cache.slab.hold(slot_b)
    assert cache.reserve(pages[3]) is None       # every rolling slot referenced: not admitted
    cache.slab.release(slot_a, None)
    assert cache.reserve(pages[3]) == slot_a
    cache.close()


def test_hot_slot_mapping_tolerates_non_contiguous_page_ids():
    layout, pages = _tiny_pages()
    pages = [replace_page(p, page_id=10 * p.page_id + 7) for p in pages]
    cache = KVPageCache(pages, layout, capacity_bytes=3 * 4096, hot_fraction=2 / 3, memory_plan=small_plan(),
                        pinned=False)
    assert cache.hot_page_ids == {7, 17}
    k = torch.zeros((16, 1, 16))
    for page in pages[:2]:
        assert not cache.get(page, k, k.clone()).hit
        cache.put(page, k, k.clone())
    for page in pages[:2]:
        assert cache.get(page, k, k.clone()).hit
    cache.close()


def test_cache_capacity_is_charged_to_the_cache_category():
    layout = KVLayout(3_145_728, 8, 128, "bf16", "bf16")
    pages = build_page_descriptors([0, 3_145_728], bytes_per_token=layout.storage_bytes_per_token,
                                   page_target_bytes=16 * 2**20, token_alignment=64)
    plan = HostMemoryPlan(total_budget_bytes=8 * 2**30, pinned_limit_bytes=1 * 2**30,
                          bounce_limit_bytes=512 * 2**20, metadata_margin_bytes=128 * 2**20)
    assert len(pages) == 384
    # Only the budgeted capacity is charged; the slab itself is not allocated
    # here (pinned=False, and the size check happens before allocation).
    records = kv_record_pages(pages, layout)
    slot = max(r.storage_bytes for r in records)
    assert plan.cache_limit_bytes // slot * slot <= plan.cache_limit_bytes


# -------------------------------------------------------------------- schedule

def test_q_groups_pack_whole_pages_and_split_large_pages():
    layout = TensorLayout(300, 2, 16, "bf16")
    pages = build_page_descriptors([0, 300], bytes_per_token=layout.bytes_per_token,
                                   page_target_bytes=64 * layout.bytes_per_token, token_alignment=16)
    groups = plan_q_groups(pages, 150)
    rows = [b.segment_start for g in groups for b in g.blocks]
    assert rows == sorted(rows)
    covered = 0
    for group in groups:
        for block in group.blocks:
            assert block.rows <= 150
            assert block.segment_start == covered
            covered += block.rows
            assert sum(p.rows for p in block.pieces) == block.rows
            assert all(p.whole_page for p in block.pieces)
    assert covered == 300
    # pages larger than a block are split into blocks of one group
    big = plan_q_groups(pages, 20)
    assert all(len(g.pages) == 1 for g in big)
    assert [b.rows for b in big[0].blocks] == [20, 20, 20, 4]
    assert [b.group_offset for b in big[0].blocks] == [0, 20, 40, 60]


def test_fragment_queue_splits_pages_across_chunks():
    queue = FragmentQueue(row_bytes=10)
    queue.push(Fragment(1000, 5000, 6, "a"))
    queue.push(Fragment(2000, 6000, 4, "b"))
    pieces, done = queue.take(8)
    assert pieces == [(1000, 5000, 6, 0, 0), (2000, 6000, 2, 0, 0)] and done == ["a"]
    pieces, done = queue.take(2)
    assert pieces == [(2020, 6020, 2, 0, 0)] and done == ["b"]
    assert queue.rows == 0
    with pytest.raises(ValueError):
        queue.take(1)


def test_fragment_queue_advances_int8_scale_rows():
    queue = FragmentQueue(row_bytes=64, scale_row_bytes=4)
    queue.push(Fragment(1000, 5000, 6, "a", ks_address=9000, vs_address=9500))
    queue.push(Fragment(2000, 6000, 4, "b", ks_address=8000, vs_address=8500))
    pieces, done = queue.take(3)
    assert pieces == [(1000, 5000, 3, 9000, 9500)] and done == []
    pieces, done = queue.take(5)
    assert pieces == [(1192, 5192, 3, 9012, 9512), (2000, 6000, 2, 8000, 8500)] and done == ["a"]
    pieces, _ = queue.take(2)
    assert pieces == [(2128, 6128, 2, 8008, 8508)]


def test_int8_slots_carry_per_row_scales():
    from seqattn.paged.cache import expand_token_scales, token_scale_layout
    from seqattn.paged.layout import KVLayout, PageDescriptor
    from seqattn.storage.records import kv_record_pages

    layout = KVLayout(total_tokens=150, heads=3, head_dim=32, source_dtype="bf16", storage_dtype="int8")
    page = PageDescriptor(page_id=0, segment_id=0, token_start=0, segment_token_start=0, valid_tokens=150,
                          padded_tokens=160)
    record = kv_record_pages([page], layout)[0]
    k_offset, v_offset, end = token_scale_layout(record, layout)
    assert k_offset >= record.storage_bytes and k_offset % 256 == 0
    assert v_offset == k_offset + 160 * 3 * 2 and end == v_offset + 160 * 3 * 2
    raw = torch.zeros(end, dtype=torch.uint8)
    groups = torch.arange(3 * 3, dtype=torch.float16).view(3, 3)  # ceil(160 / 64) groups
    raw[record.k_scale_offset : record.k_scale_offset + record.scale_bytes].view(torch.float16).copy_(groups.flatten())
    raw[record.v_scale_offset : record.v_scale_offset + record.scale_bytes].view(torch.float16).copy_(-groups.flatten())
    expand_token_scales(raw, record, layout)
    per_row_k = raw[k_offset:v_offset].view(torch.float16).view(160, 3)
    per_row_v = raw[v_offset:end].view(torch.float16).view(160, 3)
    for row in (0, 63, 64, 127, 128, 159):
        assert torch.equal(per_row_k[row], groups[row // 64])
        assert torch.equal(per_row_v[row], -groups[row // 64])
    dense = token_scale_layout(record, KVLayout(150, 3, 32, "bf16", "bf16"))
    assert dense == (0, 0, record.storage_bytes)


def test_source_contract_errors():
    q = torch.randn(17, 2, 16, dtype=torch.bfloat16)
    cu = bounds([17])
    source = MemoryPageSource(q=q, k=q, v=q, cu_seqlens_q=cu, cu_seqlens_k=cu)
    with pytest.raises(ValueError, match="storage dtype does not match"):
        validate_source_contract(source, source, cu, cu, PagedAttentionConfig(kv_storage_dtype="fp16"))
    with pytest.raises(ValueError, match="does not match q_source"):
        validate_source_contract(source, source, bounds([10, 7]), bounds([10, 7]), PagedAttentionConfig())
    keys = MemoryPageSource(k=q[:10], v=q[:10], cu_seqlens_k=bounds([0, 10]))
    queries = MemoryPageSource(q=q, cu_seqlens_q=bounds([17, 0]))
    with pytest.raises(ValueError, match="queries but no keys"):
        validate_source_contract(queries, keys, bounds([17, 0]), bounds([0, 10]), PagedAttentionConfig())
    with pytest.raises(ValueError, match="exact K/V storage dtype must match"):
        MemoryPageSource(k=q, v=q, cu_seqlens_k=cu, kv_storage_dtype="fp16")


def test_memory_sources_and_sinks():
    torch.manual_seed(223)
    q = torch.randn(97, 4, 16)
    cu = bounds([97])
    source = MemoryPageSource(q=q, k=q[:, :2].contiguous(), v=q[:, 2:].contiguous(), cu_seqlens_q=cu,
                              cu_seqlens_k=cu, page_target_bytes=2048, block_n=16)
    reader = source.open_reader(small_plan(), 1)
    page = source.q_pages[-1]
    out = torch.full((page.padded_tokens, 4, 16), 7.0)
    reader.read_q(page, out)
    assert torch.equal(out[: page.valid_tokens], q[page.token_start : page.token_stop])
    assert torch.all(out[page.valid_tokens :] == 0)
    assert source.pinned_kv_rows(0, 4) is None  # not page-locked
    result = torch.zeros_like(q)
    writer = MemoryPageSink(result).open_writer(source.q_layout, cu.tolist(), source.q_pages, small_plan(), 2)
    for p in source.q_pages:
        writer.write_page(p, q[p.token_start : p.token_stop])
    assert torch.equal(writer.close(), q)
    seen = []
    callback = CallbackOutputSink(lambda p, d: seen.append(p.page_id)).open_writer(
        source.q_layout, cu.tolist(), source.q_pages, small_plan(), 2)
    for p in source.q_pages:
        callback.write_page(p, q[p.token_start : p.token_stop])
    assert callback.close() == len(source.q_pages) == len(seen)


# -------------------------------------------------------------- on-disk stores

def make_data(dtype=torch.float32):
    torch.manual_seed(307)
    q = torch.randn(37, 4, 16, dtype=dtype)
    k = torch.randn(43, 2, 16, dtype=dtype)
    v = torch.randn_like(k)
    return q, k, v, bounds([13, 0, 24]), bounds([17, 0, 26])


def test_store_round_trip_buffered(tmp_path):
    q, k, v, cu_q, cu_k = make_data()
    store = NvmeQKVWriter.from_tensors(tmp_path / "qkv", q, k, v, cu_q, cu_k, page_target_bytes=2048,
                                       block_n=16, kv_storage_dtype="fp32", direct_io=False)
    assert NvmeQKVStore(tmp_path / "qkv", direct_io=False).kv_pages == store.kv_pages
    plan = small_plan()
    reader = store.open_reader(plan, 2)
    try:
        for page in store.q_pages:
            out = torch.empty((page.padded_tokens, 4, 16))
            reader.read_q(page, out)
            assert torch.equal(out[: page.valid_tokens], q[page.token_start : page.token_stop])
        for page in store.kv_pages:
            ko = torch.empty((page.padded_tokens, 2, 16))
            vo = torch.empty_like(ko)
            reader.read_kv(page, ko, vo)
            assert torch.equal(ko[: page.valid_tokens], k[page.token_start : page.token_stop])
            assert torch.equal(vo[: page.valid_tokens], v[page.token_start : page.token_stop])
            raw = torch.empty(page.storage_bytes, dtype=torch.uint8)
            reader.read_kv_record(page, raw)
            k_rec = raw[: page.k_bytes].view(torch.float32).view(page.padded_tokens, 2, 16)
            v_rec = raw[page.v_offset : page.v_offset + page.v_bytes].view(torch.float32).view(page.padded_tokens, 2, 16)
            assert torch.equal(k_rec[: page.valid_tokens], k[page.token_start : page.token_stop])
            assert torch.equal(v_rec[: page.valid_tokens], v[page.token_start : page.token_stop])
            assert torch.all(k_rec[page.valid_tokens :] == 0)
        # Buffered stores read rows straight into the caller's tensors: no
        # bounce memory is charged.
        assert plan.snapshot().direct_io_bounce_peak_bytes == 0
    finally:
        reader.close()
    assert plan.snapshot().direct_io_bounce_allocated_bytes == 0


def test_output_store_round_trip_and_abort(tmp_path):
    q, _, _, cu_q, _ = make_data()
    source = MemoryPageSource(q=q, cu_seqlens_q=cu_q, page_target_bytes=2048, block_n=16)
    plan = small_plan()
    writer = NvmeOutputSink(tmp_path / "out", direct_io=False).open_writer(
        source.q_layout, cu_q.tolist(), source.q_pages, plan, 2)
    for page in reversed(source.q_pages):
        writer.write_page(page, q[page.token_start : page.token_stop])
    writer.close()
    assert torch.equal(load_nvme_output(tmp_path / "out"), q)
    aborted = NvmeOutputSink(tmp_path / "aborted", direct_io=False).open_writer(
        source.q_layout, cu_q.tolist(), source.q_pages, plan, 1)
    aborted.write_page(source.q_pages[0], q[: source.q_pages[0].valid_tokens])
    aborted.abort()
    assert not (tmp_path / "aborted" / "out.bin.tmp").exists()
    assert not (tmp_path / "aborted" / "manifest.json").exists()
    assert plan.snapshot().direct_io_bounce_allocated_bytes == 0


def test_manifest_corruption_is_rejected(tmp_path):
    q, k, v, cu_q, cu_k = make_data()
    NvmeQKVWriter.from_tensors(tmp_path / "bad", q, k, v, cu_q, cu_k, page_target_bytes=2048, block_n=16,
                               kv_storage_dtype="fp32", direct_io=False)
    path = tmp_path / "bad" / "manifest.json"
    manifest = json.loads(path.read_text())
    manifest["kv_pages"][0]["token_start"] += 1
    path.write_text(json.dumps(manifest))
    with pytest.raises(ValueError, match="crosses or skips"):
        NvmeQKVStore(tmp_path / "bad", direct_io=False)
    manifest["format"] = "other"
    path.write_text(json.dumps(manifest))
    with pytest.raises(ValueError, match="unsupported or corrupt"):
        NvmeQKVStore(tmp_path / "bad", direct_io=False)


def test_short_read_is_reported(tmp_path):
    q, k, v, cu_q, cu_k = make_data()
    store = NvmeQKVWriter.from_tensors(tmp_path / "short", q, k, v, cu_q, cu_k, page_target_bytes=2048,
                                       block_n=16, kv_storage_dtype="fp32", direct_io=False)
    os.truncate(store.kv_path, store.kv_path.stat().st_size - DIRECT_IO_ALIGNMENT)
    reader = store.open_reader(small_plan(), 1)
    page = store.kv_pages[-1]
    out = torch.empty((page.padded_tokens, 2, 16))
    try:
        with pytest.raises(OSError, match="short read"):
            reader.read_kv(page, out, out.clone())
    finally:
        reader.close()


def test_direct_io_unsupported_never_falls_back(monkeypatch, tmp_path):
    path = tmp_path / "data"
    path.write_bytes(b"x" * DIRECT_IO_ALIGNMENT)
    real_open = os.open

    def reject_direct(target, flags, mode=0o777):
        if flags & getattr(os, "O_DIRECT", 0):
            raise OSError(errno.EINVAL, "not supported")
        return real_open(target, flags, mode)

    monkeypatch.setattr(os, "open", reject_direct)
    with pytest.raises(RuntimeError, match="does not support required O_DIRECT"):
        _open_file(path, os.O_RDONLY, 0, True)


def test_direct_io_round_trip_when_supported(tmp_path):
    q, k, v, cu_q, cu_k = make_data(torch.bfloat16)
    try:
        store = NvmeQKVWriter.from_tensors(tmp_path / "direct", q, k, v, cu_q, cu_k, page_target_bytes=4096,
                                           block_n=16, kv_storage_dtype="bf16", direct_io=True)
    except RuntimeError as error:
        pytest.skip(f"test filesystem has no O_DIRECT support: {error}")
    plan = small_plan()
    reader = store.open_reader(plan, 1)
    page = store.q_pages[0]
    out = torch.empty((page.padded_tokens, 4, 16), dtype=q.dtype)
    try:
        reader.read_q(page, out)
        # O_DIRECT reads go through aligned page buffers charged as bounce memory.
        assert plan.snapshot().direct_io_bounce_allocated_bytes > 0
        for kv_page in store.kv_pages:
            ko = torch.empty((kv_page.padded_tokens, 2, 16), dtype=k.dtype)
            vo = torch.empty_like(ko)
            reader.read_kv(kv_page, ko, vo)
            assert torch.equal(ko[: kv_page.valid_tokens], k[kv_page.token_start : kv_page.token_stop])
            assert torch.equal(vo[: kv_page.valid_tokens], v[kv_page.token_start : kv_page.token_stop])
    finally:
        reader.close()
    assert plan.snapshot().direct_io_bounce_allocated_bytes == 0
    assert torch.equal(out[: page.valid_tokens], q[: page.valid_tokens])


def test_disk_full_error_cleans_unpublished_store(monkeypatch, tmp_path):
    q, k, v, cu_q, cu_k = make_data()
    real = os.pwritev
    calls = 0

    def fail_after_first(fd, buffers, offset):
        nonlocal calls
        calls += 1
        if calls > 1:
            raise OSError(errno.ENOSPC, "no space left")
        return real(fd, buffers, offset)

    monkeypatch.setattr(os, "pwritev", fail_after_first)
    with pytest.raises(OSError, match="no space left"):
        NvmeQKVWriter.from_tensors(tmp_path / "full", q, k, v, cu_q, cu_k, page_target_bytes=2048, block_n=16,
                                   kv_storage_dtype="fp32", direct_io=False)
    for name in ("manifest.json", "q.bin", "kv.bin", "q.bin.tmp", "kv.bin.tmp"):
        assert not (tmp_path / "full" / name).exists()


def test_writer_rejects_wrong_pages_and_existing_store(tmp_path):
    q, k, v, cu_q, cu_k = make_data()
    writer = NvmeQKVWriter(tmp_path / "w", q_layout=TensorLayout(37, 4, 16, "fp32"),
                           kv_layout=KVLayout(43, 2, 16, "fp32", "fp32"), cu_seqlens_q=cu_q.tolist(),
                           cu_seqlens_k=cu_k.tolist(), page_target_bytes=2048, block_n=16, direct_io=False)
    with pytest.raises(ValueError, match="iterator ended early"):
        writer.write_pages(iter([]), iter([]))
    assert not (tmp_path / "w" / "q.bin.tmp").exists()
    NvmeQKVWriter.from_tensors(tmp_path / "x", q, k, v, cu_q, cu_k, page_target_bytes=2048, block_n=16,
                               direct_io=False)
    with pytest.raises(FileExistsError):
        NvmeQKVWriter.from_tensors(tmp_path / "x", q, k, v, cu_q, cu_k, direct_io=False)


# ---------------------------------------------------------------- INT8 format

def test_int8_format_matches_its_definition():
    torch.manual_seed(5)
    x = torch.randn(130, 3, 8)
    x[64:128, 1] = 0.0  # an all-zero group/head gets scale 1
    q = torch.empty(x.shape, dtype=torch.int8)
    s = torch.empty((3, 3), dtype=torch.float16)
    quantize_int8_per_token_group(x, q, s, group_tokens=64)
    assert s[1, 1] == 1.0
    for g in range(3):
        rows = slice(64 * g, min(64 * (g + 1), 130))
        amax = x[rows].abs().amax(dim=(0, 2))
        step = torch.where(amax > 0, amax / 127.0, torch.ones_like(amax))
        assert torch.equal(s[g], step.to(torch.float16))
        expected = torch.round(x[rows] / step[None, :, None]).clamp(-127, 127).to(torch.int8)
        assert torch.equal(q[rows], expected)
    back = dequantize_int8_per_token_group(q, s, dtype=torch.float32)
    # error <= half a step plus the fp16 rounding of the scale
    bound = s.float().repeat_interleave(64, 0)[:130, :, None] * (0.5 + 127 * 2**-11)
    assert torch.all((back - x).abs() <= bound + 1e-7)
    assert q.abs().max() <= 127


def test_int8_store_records_round_trip(tmp_path):
    q, k, v, cu_q, cu_k = make_data(torch.bfloat16)
    store = NvmeQKVWriter.from_tensors(tmp_path / "i8", q, k, v, cu_q, cu_k, page_target_bytes=2048,
                                       block_n=16, kv_storage_dtype="int8", direct_io=False)
    source = MemoryPageSource(q=q, k=k, v=v, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, page_target_bytes=2048,
                              block_n=16, kv_storage_dtype="int8")
    plan = small_plan()
    disk, mem = store.open_reader(plan, 1), source.open_reader(plan, 1)
    try:
        for dp, mp in zip(store.kv_pages, source.kv_pages):
            groups = math.ceil(dp.padded_tokens / 64)
            outs = [torch.empty((dp.padded_tokens, 2, 16), dtype=torch.int8) for _ in range(4)]
            scales = [torch.empty((groups, 2), dtype=torch.float16) for _ in range(4)]
            disk.read_kv(dp, outs[0], outs[1], scales[0], scales[1])
            mem.read_kv(mp, outs[2], outs[3], scales[2], scales[3])
            n = dp.valid_tokens
            g = math.ceil(n / 64)
            assert torch.equal(outs[0][:n], outs[2][:n]) and torch.equal(outs[1][:n], outs[3][:n])
            assert torch.equal(scales[0][:g], scales[2][:g]) and torch.equal(scales[1][:g], scales[3][:g])
    finally:
        disk.close()
        mem.close()
