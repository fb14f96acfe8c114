"""Python binding of libsgl_rocm_kv, the MI355X (gfx950) backend of
sglang-rs's KV-cache copy / PD-transfer path.

The names mirror the reference's Rust API so that code and tests read the
same way:

========================================  =====================================================
here                                      reference
========================================  =====================================================
``KvCacheRuntimeLayout``                  ``KvCacheRuntimeLayout`` (crates/sglang-srt/src/kv_cache.rs:57-66)
``PagedKvCacheLayout``                    ``PagedKvCacheLayout`` (kv_cache.rs:436-823)
``KvPairCopyLayout`` / ``KvPairCopyPlan`` ``CudaKvPairCopyLayout`` / ``CudaKvPairCopyPlan`` (crates/sglang-kernel/src/cuda_kv_kernels.rs:105-301)
``RocmKvPairCopyKernels``                 ``CudaKvPairCopyKernels`` (cuda_kv_kernels.rs:416-642)
``transfer_page_indices``                 ``transfer_page_indices`` (crates/sglang-srt/src/transfer.rs:679-720)
``KvError``                               ``CudaKvPairCopyError`` / ``PagedKvCacheLayoutError`` / ``KvCacheTransferPlanError``
========================================  =====================================================

``RocmKvPairCopyKernels`` adds the per-layer PD transfer calls (pack,
unpack, pool-to-pool transfer, span resolution) that the reference does not
have. Every call goes to the native library; there is no Python or CPU
fallback, and a missing library raises ``ExtensionMissing``.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libsgl_rocm_kv.so")
CODE_OBJECT_PATH = os.path.join(_HERE, "sgl_rocm_kv_gfx950.co")

# --- status codes (sgl_kv_status) ---------------------------------------------------------
OK = 0
ZERO_DIMENSION = 1
SHAPE_OVERFLOW = 2
DIMENSION_TOO_LARGE = 3
ROW_STRIDE_TOO_SMALL = 4
TENSOR_PAGE_REGION_OUT_OF_BOUNDS = 5
TENSOR_PAGE_REGIONS_OVERLAP = 6
DEVICE_MISMATCH = 7
DEVICE_SLOT_INDEX_OUT_OF_RANGE = 8
HIP = 9
MODULE = 10
ALLOCATION_OUT_OF_BOUNDS = 11
INVALID_ARGUMENT = 12
LAYOUT_ZERO_PAGE_COUNT = 20
LAYOUT_ZERO_FIELD = 21
LAYOUT_RUNTIME_PAGE_SIZE_MISMATCH = 22
LAYOUT_UNEVEN_LAYER = 23
LAYOUT_UNEVEN_TENSOR = 24
LAYOUT_SIZE_OVERFLOW = 25
LAYOUT_PAGE_OUT_OF_RANGE = 26
LAYOUT_LAYER_OUT_OF_RANGE = 27
LAYOUT_TENSOR_OUT_OF_RANGE = 28
LAYOUT_TOKEN_OUT_OF_RANGE = 29
LAYOUT_SLOT_OUT_OF_RANGE = 30
LAYOUT_EMPTY_SLOT_MAP = 31
LAYOUT_BATCH_SLOT_OUT_OF_RANGE = 32
LAYOUT_KV_PAIR_REQUIRES_TWO_TENSORS = 33
LAYOUT_TENSOR_PAIR_REQUIRES_TWO_TENSORS = 34
LAYOUT_TENSOR_PAIR_SIZE_MISMATCH = 35
LAYOUT_UNEVEN_KV_PAIR_COPY = 36
PLAN_ZERO_PAGE_SIZE = 40
PLAN_UNALIGNED_TOKEN_OFFSET = 43
PLAN_UNALIGNED_CACHE_SLOT = 44
PLAN_NON_CONTIGUOUS_CACHE_SLOTS = 45
PLAN_NON_PREFILL_BATCH = 46
PLAN_CACHE_PAGE_COUNT_MISMATCH = 41
PLAN_TRAILING_CACHE_PAGES = 42
RADIX_TOKEN_PAGE_LENGTH_MISMATCH = 74
FORWARD_PREFILL, FORWARD_DECODE = 0, 1
DEVICE_PAGE_INDEX_OUT_OF_RANGE = 50
DEVICE_SPAN_OUT_OF_RANGE = 51
DEVICE_REQUEST_OUT_OF_RANGE = 52
STORAGE_SIZE_MISMATCH = 110
STORAGE_SLOT_MAP_CAPACITY_MISMATCH = 111
STORAGE_PAGE_BUFFER_SIZE_MISMATCH = 112
STORAGE_SIZE_OVERFLOW = 113
ZERO_ALLOCATION = 114
UNSUPPORTED_MEMORY_LOCATION = 115
STORAGE_DESCRIPTOR = 116
# KvCacheMemoryLocation kinds (sgl_kv_memory_location_kind)
LOCATION_CPU, LOCATION_CUDA, LOCATION_ROCM, LOCATION_MUSA = 0, 1, 2, 3
LOCATION_NPU, LOCATION_METAL, LOCATION_XPU, LOCATION_HPU = 4, 5, 6, 7

DTYPES = {"auto": 0, "float32": 1, "bf16": 2, "bfloat16": 2, "fp8_e4m3": 3, "fp8_e5m2": 4,
          "fp4_e2m1": 5}
NHD, HND = 0, 1
# Attention plan flags (no counterpart in the reference): hi + lo bf16
# softmax weights are the default in every body (EXACT names it); FAST lets
# the latent (MLA) body round each weight to one bf16 instead.
ATTN_EXACT_WEIGHTS = 1
ATTN_FAST_WEIGHTS = 2
FILL_BITS, FILL_BF16_NORMAL, FILL_BF16_UNIFORM = 0, 1, 2
STREAM_COPY, STREAM_READ, STREAM_WRITE = 0, 1, 2


class ExtensionMissing(RuntimeError):
    """The native library or its gfx950 code object has not been built."""


class KvError(Exception):
    """A failed call: ``code`` (sgl_kv_status), ``variant`` (the reference's
    error variant name), ``name`` and ``fields`` (a, b, c) of the variant."""

    def __init__(self, code, variant, name, fields, message):
        super().__init__(f"{variant}: {message}")
        self.code, self.variant, self.name, self.fields, self.message = (
            code, variant, name, fields, message)


# --- C structs (field for field as include/sgl_rocm_kv.h) ------------------------------------
_u64 = ctypes.c_uint64


class _ErrorDetail(ctypes.Structure):
    _fields_ = [("code", ctypes.c_int32), ("reserved", ctypes.c_int32), ("a", _u64), ("b", _u64),
                ("c", _u64), ("d", _u64), ("name", ctypes.c_char * 64),
                ("message", ctypes.c_char * 320)]


class _RuntimeLayout(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int32), ("reserved", ctypes.c_int32)] + [
        (n, _u64) for n in ("page_size", "num_layers", "kv_heads", "head_dim",
                            "kv_tensors_per_token", "bytes_per_token", "page_size_bytes")]


class _ModelLayout(ctypes.Structure):
    _fields_ = [(n, _u64) for n in ("num_layers", "kv_heads", "head_dim", "kv_tensors_per_token",
                                    "bytes_per_token_per_layer")] + [
        ("geometry", ctypes.c_uint32), ("reserved", ctypes.c_uint32),
        ("key_elements", _u64), ("value_elements", _u64)]


class _PagedLayout(ctypes.Structure):
    _fields_ = [("runtime", _RuntimeLayout), ("page_count", _u64),
                ("bytes_per_token_per_layer", _u64), ("bytes_per_layer_page", _u64),
                ("tensor_pair", _u64), ("token_bytes", _u64 * 2), ("tensor_page_bytes", _u64),
                ("total_byte_len", _u64), ("slot_count", _u64)]


class _PairCopyLayout(ctypes.Structure):
    _fields_ = [(n, _u64) for n in ("page_size", "page_stride_bytes", "key_in_page_offset",
                                    "value_in_page_offset", "row_bytes")]


class _PairCopyPlan(ctypes.Structure):
    _fields_ = [("row_count", _u64), ("slot_count", _u64), ("layout", _PairCopyLayout)] + [
        (n, _u64) for n in ("key_row_stride_bytes", "value_row_stride_bytes",
                            "key_rows_required_bytes", "value_rows_required_bytes",
                            "slot_indices_required_bytes", "pool_required_bytes")]


class _DeviceBuffer(ctypes.Structure):
    _fields_ = [("ptr", ctypes.c_void_p), ("byte_len", _u64)]


class _FramePart(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("len", _u64)]


class _DecodeLayout(ctypes.Structure):
    _fields_ = [("layout", _PagedLayout), ("head_layout", ctypes.c_uint32), ("reserved", ctypes.c_uint32),
                ("heads", _u64)]


def _lists_struct(ct):
    class L(ctypes.Structure):
        _fields_ = [("values", ctypes.POINTER(ct)), ("offsets", ctypes.POINTER(_u64)), ("count", _u64)]
    return L


_U64Lists, _U32Lists, _I32Lists = _lists_struct(_u64), _lists_struct(ctypes.c_uint32), _lists_struct(ctypes.c_int32)


class _BootKvArgs(ctypes.Structure):
    _fields_ = [("endpoint", ctypes.c_char_p), ("mooncake_session_id", ctypes.c_char_p),
                ("dst_port", ctypes.c_uint32), ("dst_tp_rank", ctypes.c_int32),
                ("dst_attn_tp_size", _u64), ("dst_kv_item_len", _u64),
                ("dst_kv_ptrs", ctypes.POINTER(_u64)), ("dst_kv_ptr_count", _u64),
                ("dst_aux_ptrs", ctypes.POINTER(_u64)), ("dst_aux_ptr_count", _u64),
                ("dst_state_data_ptrs", _U64Lists), ("dst_state_item_lens", _U32Lists),
                ("dst_state_dim_per_tensor", _U32Lists), ("decode_layout", ctypes.POINTER(_DecodeLayout))]


class _BootTransfer(ctypes.Structure):
    _fields_ = [("room", _u64), ("endpoint", ctypes.c_char_p), ("mooncake_session_id", ctypes.c_char_p),
                ("dst_port", ctypes.c_uint32), ("is_dummy", ctypes.c_uint32),
                ("dst_kv_indices", ctypes.POINTER(ctypes.c_int32)), ("dst_kv_index_count", _u64),
                ("has_dst_aux_index", ctypes.c_uint32), ("dst_aux_index", ctypes.c_int32),
                ("dst_state_indices", _I32Lists), ("required_dst_info_num", _u64),
                ("has_decode_prefix_len", ctypes.c_uint32), ("reserved", ctypes.c_uint32),
                ("decode_prefix_len", _u64)]


class _RemoteKvLayout(ctypes.Structure):
    _fields_ = [("mooncake_session_id", ctypes.c_char_p),
                ("dst_kv_ptrs", ctypes.POINTER(_u64)), ("dst_kv_ptr_count", _u64),
                ("dst_kv_indices", ctypes.POINTER(ctypes.c_int32)), ("dst_kv_index_count", _u64),
                ("dst_kv_item_len", _u64), ("decode_layout", ctypes.POINTER(_DecodeLayout))]


class _PairCopyBuffers(ctypes.Structure):
    _fields_ = [("keys", _DeviceBuffer), ("keys_offset", _u64), ("values", _DeviceBuffer),
                ("values_offset", _u64), ("slot_indices", _DeviceBuffer),
                ("slot_indices_offset", _u64), ("pool", _DeviceBuffer), ("pool_offset", _u64)]


class PoolView(ctypes.Structure):
    """sgl_kv_pool_view: one layer of a page-major pool on the device."""
    _fields_ = [("base", ctypes.c_void_p), ("byte_len", _u64), ("page_size", _u64),
                ("page_stride_bytes", _u64), ("page_count", _u64), ("tensor_offset", _u64 * 2),
                ("row_bytes", _u64), ("tensor_count", ctypes.c_uint32),
                ("heads", ctypes.c_uint32), ("head_layout", ctypes.c_uint32),
                ("reserved", ctypes.c_uint32), ("scale", ctypes.c_void_p),
                ("value_row_bytes", _u64)]

    def tensor_row_bytes(self, tensor: int) -> int:
        """Bytes per (token, tensor): the value width of a tensor pair may differ."""
        return self.value_row_bytes if tensor == 1 and self.value_row_bytes else self.row_bytes


class RowsView(ctypes.Structure):
    """sgl_kv_rows_view: contiguous transfer rows, planes[t] + r * row_stride[t]."""
    _fields_ = [("planes", ctypes.c_void_p * 2), ("plane_bytes", _u64 * 2),
                ("row_stride", _u64 * 2), ("scale", ctypes.c_void_p)]


class _PipelineDesc(ctypes.Structure):
    _fields_ = [("layers", ctypes.c_uint32), ("staged", ctypes.c_uint32),
                ("src_layers", ctypes.POINTER(PoolView)), ("dst_layers", ctypes.POINTER(PoolView)),
                ("src_slots", _DeviceBuffer), ("dst_slots", _DeviceBuffer), ("row_count", _u64),
                ("send", _DeviceBuffer * 2), ("recv", _DeviceBuffer * 2),
                ("host", ctypes.c_void_p * 2), ("host_bytes", _u64)]


class _BackendConfig(ctypes.Structure):
    _fields_ = [("mode", ctypes.c_uint32), ("reserved", ctypes.c_uint32), ("max_rows", _u64)]


class _BackendMemory(ctypes.Structure):
    _fields_ = [("layout", _PagedLayout), ("base", ctypes.c_void_p), ("byte_len", _u64),
                ("head_layout", ctypes.c_uint32), ("reserved", ctypes.c_uint32), ("heads", _u64)]


class _TensorLocation(ctypes.Structure):
    _fields_ = [("device_ptr", _u64), ("byte_offset", _u64), ("byte_len", _u64)]


class _SlotRows(ctypes.Structure):
    _fields_ = [("keys", _DeviceBuffer), ("keys_offset", _u64), ("key_row_stride_bytes", _u64),
                ("values", _DeviceBuffer), ("values_offset", _u64), ("value_row_stride_bytes", _u64)]


class _MemoryRegion(ctypes.Structure):
    _fields_ = [("base_addr", _u64), ("byte_len", _u64), ("page_size_bytes", _u64)]


MAX_MEMORY_REGIONS = 8


class _TransferableMemory(ctypes.Structure):
    _fields_ = [("regions", _MemoryRegion * MAX_MEMORY_REGIONS), ("region_count", _u64),
                ("page_size_bytes", _u64), ("location_kind", ctypes.c_int32), ("location_id", ctypes.c_int32)]


PLACEMENT_MAX_CANDIDATES = 8


class _PlacementReport(ctypes.Structure):
    _fields_ = [("candidates", ctypes.c_uint32), ("chosen", ctypes.c_uint32), ("probe_rows", _u64),
                ("probe_us", ctypes.c_float * PLACEMENT_MAX_CANDIDATES)]


class _SpanDesc(ctypes.Structure):
    _fields_ = [("bootstrap_room", _u64), ("descriptor_checksum", ctypes.c_char * 65),
                ("reserved", ctypes.c_char * 7), ("token_offset", _u64), ("token_count", _u64),
                ("cache_slots", ctypes.POINTER(_u64)),
                ("dst_page_table", ctypes.POINTER(ctypes.c_int32)),
                ("dst_page_table_len", _u64)]


class _TransferEvent(ctypes.Structure):
    _fields_ = [("bootstrap_room", _u64), ("descriptor_checksum", ctypes.c_char * 65),
                ("reserved", ctypes.c_char * 3), ("status", ctypes.c_int32),
                ("error_code", ctypes.c_int32)]


class _AttentionLayout(ctypes.Structure):
    _fields_ = [(n, _u64) for n in ("page_size", "page_stride_bytes", "key_in_page_offset",
                                    "value_in_page_offset", "key_row_bytes", "value_row_bytes")] + [
        ("head_layout", ctypes.c_uint32), ("reserved", ctypes.c_uint32)]


class _AttentionPlanConfig(ctypes.Structure):
    _fields_ = [(n, _u64) for n in ("query_count", "request_count", "sequence_slot_count",
                                    "slot_count", "query_head_count", "kv_head_count",
                                    "query_key_head_dim", "value_head_dim")] + [
        ("scale", ctypes.c_float), ("flags", ctypes.c_uint32), ("layout", _AttentionLayout)]


_ATTENTION_REQUIRED = ("query_required_bytes", "query_request_indices_required_bytes",
                       "query_sequence_lengths_required_bytes",
                       "request_slot_offsets_required_bytes", "sequence_slots_required_bytes",
                       "pool_required_bytes", "output_required_bytes")


class _AttentionPlan(ctypes.Structure):
    _fields_ = [("config", _AttentionPlanConfig)] + [(n, _u64) for n in _ATTENTION_REQUIRED]


_ATTENTION_BUFFERS = ("queries", "query_request_indices", "query_sequence_lengths",
                      "request_slot_offsets", "sequence_slots", "pool", "output")


class _AttentionBuffers(ctypes.Structure):
    _fields_ = [f for n in _ATTENTION_BUFFERS for f in ((n, _DeviceBuffer), (n + "_offset", _u64))]


PAGE_REQUEST_DTYPE = np.dtype([("source", "<u8"), ("target_offset", "<u8"), ("length", "<u8")])


# sgl_kv_plan_span: one KvCacheTransferSpan as offsets into the batch and
# the plan's page-index array.
PLAN_SPAN_DTYPE = np.dtype([("request_index", "<u8"), ("token_offset", "<u8"), ("token_count", "<u8"),
                            ("cache_page_offset", "<u8"), ("page_index_offset", "<u8"),
                            ("page_index_count", "<u8")])


class _PrefillBatch(ctypes.Structure):
    _fields_ = [("forward_mode", ctypes.c_int32), ("request_count", ctypes.c_uint64),
                ("input_token_counts", ctypes.POINTER(ctypes.c_uint64)),
                ("cached_token_counts", ctypes.POINTER(ctypes.c_uint64)),
                ("has_disaggregated_params", ctypes.POINTER(ctypes.c_uint8)),
                ("out_cache_pages", ctypes.POINTER(ctypes.c_uint64)),
                ("out_cache_page_count", ctypes.c_uint64)]


SPAN_DTYPE = np.dtype([("row_start", "<u4"), ("token_offset", "<u4"), ("token_count", "<u4"),
                       ("page_table_start", "<u4")])

_EXPORTS = {
    "sgl_kv_last_error": (None, [ctypes.POINTER(_ErrorDetail)]),
    "sgl_kv_status_name": (ctypes.c_char_p, [ctypes.c_int32]),
    "sgl_kv_dtype_bytes_per_element": (ctypes.c_size_t, [ctypes.c_int32]),
    "sgl_kv_model_layout_multi_tensor": (ctypes.c_int32, [_u64, _u64, _u64, _u64, ctypes.POINTER(_ModelLayout)]),
    "sgl_kv_model_layout_tensor_pair": (ctypes.c_int32, [_u64, _u64, _u64, _u64, _u64,
                                                         ctypes.POINTER(_ModelLayout)]),
    "sgl_kv_model_layout_packed_bytes_per_layer": (ctypes.c_int32, [_u64, _u64, ctypes.POINTER(_ModelLayout)]),
    "sgl_kv_model_layout_packed_mla": (ctypes.c_int32, [_u64, _u64, _u64, ctypes.POINTER(_ModelLayout)]),
    "sgl_kv_model_layout_elements_per_token": (ctypes.c_int32, [ctypes.POINTER(_ModelLayout), ctypes.POINTER(_u64),
                                                                ctypes.POINTER(ctypes.c_uint32)]),
    "sgl_kv_model_layout_token_size_bytes": (ctypes.c_int32, [ctypes.POINTER(_ModelLayout), ctypes.c_int32,
                                                              ctypes.POINTER(_u64)]),
    "sgl_kv_model_layout_tensor_pair_size_bytes": (ctypes.c_int32, [ctypes.POINTER(_ModelLayout), ctypes.c_int32,
                                                                    _u64 * 2, ctypes.POINTER(ctypes.c_uint32)]),
    "sgl_kv_paged_layout_for_model": (ctypes.c_int32, [ctypes.POINTER(_ModelLayout), ctypes.c_int32, _u64, _u64,
                                                       ctypes.POINTER(_PagedLayout)]),
    "sgl_kv_paged_layout_new": (ctypes.c_int32, [ctypes.POINTER(_RuntimeLayout), _u64,
                                                 ctypes.POINTER(_PagedLayout)]),
    "sgl_kv_paged_layout_new_with_tensor_pair": (
        ctypes.c_int32, [ctypes.POINTER(_RuntimeLayout), _u64, _u64, _u64,
                         ctypes.POINTER(_PagedLayout)]),
    "sgl_kv_paged_layout_page_byte_range": (
        ctypes.c_int32, [ctypes.POINTER(_PagedLayout), _u64, ctypes.POINTER(_u64),
                         ctypes.POINTER(_u64)]),
    "sgl_kv_paged_layout_tensor_token_byte_range": (
        ctypes.c_int32, [ctypes.POINTER(_PagedLayout), _u64, _u64, _u64, _u64,
                         ctypes.POINTER(_u64), ctypes.POINTER(_u64)]),
    "sgl_kv_paged_layout_tensor_slot_byte_range": (
        ctypes.c_int32, [ctypes.POINTER(_PagedLayout), _u64, _u64, _u64, ctypes.POINTER(_u64),
                         ctypes.POINTER(_u64)]),
    "sgl_kv_paged_layout_validate_slot_indices": (
        ctypes.c_int32, [ctypes.POINTER(_PagedLayout), ctypes.POINTER(_u64), _u64]),
    "sgl_kv_paged_layout_kv_pair_copy_geometry": (
        ctypes.c_int32, [ctypes.POINTER(_PagedLayout), _u64, ctypes.POINTER(_PairCopyLayout)]),
    "sgl_kv_pair_copy_plan_new": (
        ctypes.c_int32, [_u64, _u64, ctypes.POINTER(_PairCopyLayout), _u64, _u64,
                         ctypes.POINTER(_PairCopyPlan)]),
    "sgl_kv_transfer_page_indices": (
        ctypes.c_int32, [_u64, _u64, ctypes.POINTER(_u64), _u64, _u64, ctypes.POINTER(_u64),
                         ctypes.POINTER(_u64)]),
    "sgl_kv_pool_view_for_layer": (
        ctypes.c_int32, [ctypes.POINTER(_PagedLayout), ctypes.c_void_p, _u64, ctypes.c_uint32,
                         _u64, _u64, _u64, _u64, ctypes.POINTER(PoolView)]),
    "sgl_kv_build_page_requests": (
        ctypes.c_int32, [_u64, _u64, _u64, _u64, _u64, _u64, ctypes.POINTER(_u64), _u64,
                         ctypes.c_void_p, _u64, ctypes.POINTER(_u64)]),
    "sgl_kv_build_remote_page_requests": (
        ctypes.c_int32, [_u64, _u64, _u64, _u64, ctypes.POINTER(_u64), _u64, ctypes.POINTER(_u64),
                         _u64, ctypes.POINTER(ctypes.c_int32), _u64, _u64, ctypes.c_void_p, _u64,
                         ctypes.POINTER(_u64)]),
    "sgl_kv_page_allocator_new": (ctypes.c_int32, [_u64, _u64, ctypes.POINTER(ctypes.c_void_p)]),
    "sgl_kv_page_allocator_destroy": (ctypes.c_int32, [ctypes.c_void_p]),
    "sgl_kv_page_allocator_available_pages": (_u64, [ctypes.c_void_p]),
    "sgl_kv_page_allocator_available_slots": (_u64, [ctypes.c_void_p]),
    "sgl_kv_page_allocator_allocate_for_sequence": (
        ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(_u64), _u64, _u64, ctypes.POINTER(_u64)]),
    "sgl_kv_page_allocator_release": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(_u64), _u64]),
    "sgl_kv_page_allocator_reset": (ctypes.c_int32, [ctypes.c_void_p]),
    "sgl_kv_radix_cache_new": (ctypes.c_int32, [ctypes.POINTER(ctypes.c_void_p)]),
    "sgl_kv_radix_cache_destroy": (ctypes.c_int32, [ctypes.c_void_p]),
    "sgl_kv_radix_cache_clear": (ctypes.c_int32, [ctypes.c_void_p]),
    "sgl_kv_radix_cache_insert": (
        ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint32), _u64, ctypes.POINTER(_u64), _u64]),
    "sgl_kv_radix_cache_match_prefix": (
        ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint32), _u64, _u64, ctypes.POINTER(_u64),
                         ctypes.POINTER(_u64)]),
    "sgl_kv_transfer_plan_from_prefill_batch": (
        ctypes.c_int32, [ctypes.POINTER(_PrefillBatch), _u64, ctypes.c_void_p, _u64, ctypes.POINTER(_u64), _u64,
                         ctypes.POINTER(_u64), ctypes.POINTER(_u64)]),
    "sgl_kv_transfer_span_checksum": (
        ctypes.c_int32, [ctypes.c_char_p, _u64, ctypes.c_char_p, _u64, ctypes.c_uint16, _u64,
                         ctypes.c_int32, _u64, _u64, _u64, ctypes.POINTER(_u64), _u64,
                         ctypes.POINTER(_u64), _u64, ctypes.c_char_p]),
    "sgl_kv_sha256_hex": (ctypes.c_int32, [ctypes.c_char_p, _u64, ctypes.c_char_p]),
    "sgl_rocm_kv_init": (ctypes.c_int32, [ctypes.c_int32, ctypes.c_char_p,
                                          ctypes.POINTER(ctypes.c_void_p)]),
    "sgl_rocm_kv_destroy": (ctypes.c_int32, [ctypes.c_void_p]),
    "sgl_rocm_kv_device": (ctypes.c_int32, [ctypes.c_void_p]),
    "sgl_rocm_kv_cu_count": (ctypes.c_int32, [ctypes.c_void_p]),
    "sgl_rocm_kv_pair_scatter": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(_PairCopyPlan),
                                                  ctypes.POINTER(_PairCopyBuffers),
                                                  ctypes.c_void_p]),
    "sgl_rocm_kv_pair_gather": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(_PairCopyPlan),
                                                 ctypes.POINTER(_PairCopyBuffers),
                                                 ctypes.c_void_p]),
    "sgl_rocm_kv_pack_layer": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(PoolView),
                                                ctypes.POINTER(_DeviceBuffer), _u64,
                                                ctypes.POINTER(RowsView), ctypes.c_void_p]),
    "sgl_rocm_kv_unpack_layer": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(RowsView), _u64,
                                                  ctypes.POINTER(PoolView),
                                                  ctypes.POINTER(_DeviceBuffer), ctypes.c_void_p]),
    "sgl_rocm_kv_pack_layers": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(PoolView), _u64,
                                                 ctypes.c_uint32, ctypes.POINTER(_DeviceBuffer), _u64,
                                                 ctypes.POINTER(RowsView), _u64, ctypes.c_void_p]),
    "sgl_rocm_kv_unpack_layers": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(RowsView), _u64,
                                                   ctypes.c_uint32, _u64, ctypes.POINTER(PoolView),
                                                   _u64, ctypes.POINTER(_DeviceBuffer),
                                                   ctypes.c_void_p]),
    "sgl_rocm_kv_write_tensor_slots": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(_PagedLayout),
                                                        ctypes.POINTER(_DeviceBuffer), _u64, _u64,
                                                        ctypes.POINTER(_DeviceBuffer), _u64,
                                                        ctypes.POINTER(_DeviceBuffer), _u64, _u64,
                                                        ctypes.c_void_p]),
    "sgl_rocm_kv_write_tensor_pair_slots": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(_PagedLayout),
                                                             ctypes.POINTER(_DeviceBuffer), _u64,
                                                             ctypes.POINTER(_DeviceBuffer), _u64,
                                                             ctypes.POINTER(_DeviceBuffer), _u64, _u64,
                                                             ctypes.POINTER(_DeviceBuffer), _u64, _u64,
                                                             ctypes.c_void_p]),
    "sgl_rocm_kv_read_tensor_slots": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(_PagedLayout),
                                                       ctypes.POINTER(_DeviceBuffer), _u64, _u64,
                                                       ctypes.POINTER(_DeviceBuffer), _u64,
                                                       ctypes.POINTER(_DeviceBuffer), _u64, _u64,
                                                       ctypes.c_void_p]),
    "sgl_rocm_kv_transfer_layers": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(PoolView), _u64,
                                                     ctypes.c_uint32, ctypes.POINTER(_DeviceBuffer),
                                                     _u64, ctypes.POINTER(PoolView), _u64,
                                                     ctypes.POINTER(_DeviceBuffer), ctypes.c_void_p]),
    "sgl_rocm_kv_transfer_layer": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(PoolView),
                                                    ctypes.POINTER(_DeviceBuffer), _u64,
                                                    ctypes.POINTER(PoolView),
                                                    ctypes.POINTER(_DeviceBuffer),
                                                    ctypes.c_void_p]),
    "sgl_rocm_kv_resolve_spans": (ctypes.c_int32, [ctypes.c_void_p, _u64, _u64,
                                                   ctypes.POINTER(_DeviceBuffer), _u64,
                                                   ctypes.POINTER(_DeviceBuffer), _u64, _u64,
                                                   ctypes.POINTER(_DeviceBuffer),
                                                   ctypes.c_void_p]),
    "sgl_rocm_kv_check_errors": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_void_p]),
    "sgl_rocm_kv_pipeline_create": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(_PipelineDesc),
                                                     ctypes.POINTER(ctypes.c_void_p)]),
    "sgl_rocm_kv_pipeline_run": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_void_p]),
    "sgl_rocm_kv_pipeline_wait": (ctypes.c_int32, [ctypes.c_void_p]),
    "sgl_rocm_kv_pipeline_layer_times": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_uint32,
                                                          ctypes.POINTER(ctypes.c_float)]),
    "sgl_rocm_kv_pipeline_elapsed": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_float)]),
    "sgl_rocm_kv_pipeline_destroy": (ctypes.c_int32, [ctypes.c_void_p]),
    "sgl_rocm_kv_backend_create": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(_BackendConfig),
                                                    ctypes.POINTER(ctypes.c_void_p)]),
    "sgl_rocm_kv_backend_register": (ctypes.c_int32, [ctypes.c_void_p,
                                                      ctypes.POINTER(_BackendMemory),
                                                      ctypes.POINTER(_BackendMemory)]),
    "sgl_rocm_kv_backend_submit": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(_SpanDesc)]),
    "sgl_rocm_kv_backend_submit_device_table": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(_SpanDesc)]),
    "sgl_rocm_kv_backend_poll": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(_TransferEvent),
                                                  _u64, ctypes.POINTER(_u64), ctypes.POINTER(_u64)]),
    "sgl_rocm_kv_backend_cancel": (ctypes.c_int32, [ctypes.c_void_p, _u64]),
    "sgl_rocm_kv_backend_wait": (ctypes.c_int32, [ctypes.c_void_p]),
    "sgl_rocm_kv_backend_shutdown": (ctypes.c_int32, [ctypes.c_void_p]),
    "sgl_rocm_kv_backend_destroy": (ctypes.c_int32, [ctypes.c_void_p]),
    "sgl_kv_attention_plan_new": (ctypes.c_int32, [ctypes.POINTER(_AttentionPlanConfig),
                                                   ctypes.POINTER(_AttentionPlan)]),
    "sgl_kv_attention_plan_for_layer": (ctypes.c_int32, [ctypes.POINTER(_PagedLayout), _u64, _u64,
                                                         _u64, _u64, _u64, ctypes.c_float,
                                                         ctypes.c_uint32,
                                                         ctypes.POINTER(_AttentionPlan)]),
    "sgl_rocm_kv_paged_attention": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(_AttentionPlan),
                                                     ctypes.POINTER(_AttentionBuffers), _u64,
                                                     ctypes.c_void_p]),
    "sgl_rocm_kv_paged_attention_async": (ctypes.c_int32, [ctypes.c_void_p,
                                                           ctypes.POINTER(_AttentionPlan),
                                                           ctypes.POINTER(_AttentionBuffers), _u64,
                                                           ctypes.c_void_p]),
    "sgl_rocm_kv_paged_attention_async_noalloc": (ctypes.c_int32, [ctypes.c_void_p,
                                                                   ctypes.POINTER(_AttentionPlan),
                                                                   ctypes.POINTER(_AttentionBuffers), _u64,
                                                                   ctypes.c_void_p]),
    "sgl_rocm_kv_execute_page_requests": (ctypes.c_int32, [ctypes.c_void_p,
                                                           ctypes.POINTER(_DeviceBuffer), _u64, _u64,
                                                           ctypes.POINTER(_DeviceBuffer),
                                                           ctypes.POINTER(_DeviceBuffer),
                                                           ctypes.c_uint32, ctypes.c_void_p]),
    "sgl_rocm_kv_fill_synthetic": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(_DeviceBuffer),
                                                    _u64, ctypes.c_uint32, ctypes.c_void_p]),
    "sgl_rocm_kv_stream": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_uint32, ctypes.POINTER(_DeviceBuffer),
                                            ctypes.POINTER(_DeviceBuffer), _u64, ctypes.c_void_p]),
    "sgl_rocm_kv_memory_info": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(_u64), ctypes.POINTER(_u64)]),
    "sgl_rocm_kv_storage_allocate": (ctypes.c_int32, [ctypes.c_void_p, _u64, _u64, ctypes.POINTER(ctypes.c_void_p)]),
    "sgl_rocm_kv_cache_allocate": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(_RuntimeLayout), _u64,
                                                    ctypes.POINTER(_PagedLayout), ctypes.POINTER(ctypes.c_void_p)]),
    "sgl_rocm_kv_pool_allocate": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(_PagedLayout),
                                                   ctypes.POINTER(ctypes.c_void_p)]),
    "sgl_rocm_kv_storage_allocate_placed": (ctypes.c_int32, [ctypes.c_void_p, _u64, _u64, ctypes.POINTER(PoolView),
                                                             ctypes.POINTER(_DeviceBuffer), ctypes.POINTER(PoolView),
                                                             ctypes.c_uint32,
                                                             ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p),
                                                             ctypes.POINTER(_PlacementReport)]),
    "sgl_rocm_kv_storage_destroy": (ctypes.c_int32, [ctypes.c_void_p]),
    "sgl_rocm_kv_storage_allocation": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(_DeviceBuffer)]),
    "sgl_rocm_kv_storage_byte_len": (_u64, [ctypes.c_void_p]),
    "sgl_rocm_kv_storage_page_size_bytes": (_u64, [ctypes.c_void_p]),
    "sgl_rocm_kv_storage_device": (ctypes.c_int32, [ctypes.c_void_p]),
    "sgl_rocm_kv_storage_clear": (ctypes.c_int32, [ctypes.c_void_p]),
    "sgl_rocm_kv_storage_validate_layout": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(_PagedLayout)]),
    "sgl_rocm_kv_storage_write_page": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(_PagedLayout), _u64,
                                                        ctypes.c_void_p, _u64]),
    "sgl_rocm_kv_storage_read_page": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(_PagedLayout), _u64,
                                                       ctypes.c_void_p, _u64]),
    "sgl_rocm_kv_storage_write_tensor_slot": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(_PagedLayout), _u64,
                                                               _u64, _u64, ctypes.POINTER(_DeviceBuffer), _u64,
                                                               ctypes.c_void_p]),
    "sgl_rocm_kv_storage_read_tensor_slot": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(_PagedLayout), _u64,
                                                              _u64, _u64, ctypes.POINTER(_DeviceBuffer), _u64,
                                                              ctypes.c_void_p]),
    "sgl_rocm_kv_storage_tensor_location": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(_PagedLayout), _u64,
                                                             _u64, _u64, _u64, ctypes.POINTER(_TensorLocation)]),
    "sgl_rocm_kv_storage_slot_location": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(_PagedLayout), _u64,
                                                           _u64, _u64, ctypes.POINTER(_TensorLocation)]),
    "sgl_rocm_kv_storage_upload_slot_map": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(_PagedLayout),
                                                             ctypes.POINTER(_u64), _u64,
                                                             ctypes.POINTER(ctypes.c_void_p)]),
    "sgl_rocm_kv_slot_map_destroy": (ctypes.c_int32, [ctypes.c_void_p]),
    "sgl_rocm_kv_slot_map_allocation": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(_DeviceBuffer)]),
    "sgl_rocm_kv_slot_map_len": (_u64, [ctypes.c_void_p]),
    "sgl_rocm_kv_slot_map_slots": (ctypes.POINTER(_u64), [ctypes.c_void_p]),
    "sgl_rocm_kv_storage_write_kv_slots": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_void_p,
                                                            ctypes.POINTER(_PagedLayout), _u64, ctypes.c_void_p,
                                                            ctypes.POINTER(_SlotRows), ctypes.c_void_p]),
    "sgl_rocm_kv_storage_read_kv_slots": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_void_p,
                                                           ctypes.POINTER(_PagedLayout), _u64, ctypes.c_void_p,
                                                           ctypes.POINTER(_SlotRows), ctypes.c_void_p]),
    "sgl_rocm_kv_storage_transferable_memory": (ctypes.c_int32, [ctypes.c_void_p,
                                                                 ctypes.POINTER(_TransferableMemory)]),
    "sgl_rocm_kv_storage_backend_memory": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(_PagedLayout),
                                                            ctypes.c_uint32, _u64, ctypes.POINTER(_BackendMemory)]),
    "sgl_kv_memory_location_label": (ctypes.c_int32, [ctypes.c_int32, ctypes.c_int32, ctypes.c_char * 32]),
    "sgl_kv_transferable_memory_decode_remote_layout": (ctypes.c_int32, [ctypes.POINTER(_TransferableMemory),
                                                                         ctypes.POINTER(_u64), _u64,
                                                                         ctypes.POINTER(_u64),
                                                                         ctypes.POINTER(_u64)]),
    "sgl_kv_bootstrap_create": (ctypes.c_int32, [ctypes.POINTER(ctypes.c_void_p)]),
    "sgl_kv_bootstrap_destroy": (ctypes.c_int32, [ctypes.c_void_p]),
    "sgl_kv_bootstrap_ingest": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(_FramePart), ctypes.c_uint32]),
    "sgl_kv_bootstrap_registration_count": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(_u64)]),
    "sgl_kv_bootstrap_get_kv_args": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_char_p,
                                                      ctypes.POINTER(_BootKvArgs)]),
    "sgl_kv_bootstrap_transfer_status": (ctypes.c_int32, [ctypes.c_void_p, _u64, ctypes.POINTER(ctypes.c_int32)]),
    "sgl_kv_bootstrap_room": (ctypes.c_int32, [ctypes.c_void_p, _u64, ctypes.POINTER(_u64),
                                               ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(_u64),
                                               ctypes.POINTER(_u64)]),
    "sgl_kv_bootstrap_get_transfer": (ctypes.c_int32, [ctypes.c_void_p, _u64, ctypes.c_char_p,
                                                       ctypes.POINTER(_BootTransfer)]),
    "sgl_kv_bootstrap_remote_layouts": (ctypes.c_int32, [ctypes.c_void_p, _u64, ctypes.POINTER(_RemoteKvLayout),
                                                         _u64, ctypes.POINTER(_u64)]),
    "sgl_kv_bootstrap_encode_kv_args": (ctypes.c_int32, [ctypes.POINTER(_BootKvArgs), ctypes.c_void_p, _u64,
                                                         ctypes.POINTER(_FramePart),
                                                         ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(_u64)]),
    "sgl_kv_bootstrap_encode_transfer": (ctypes.c_int32, [ctypes.POINTER(_BootTransfer), ctypes.c_void_p, _u64,
                                                          ctypes.POINTER(_FramePart),
                                                          ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(_u64)]),
}

_lib = None


def lib():
    """The loaded native library; raises ExtensionMissing when it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ExtensionMissing(
                f"{LIB_PATH} is not built: run `python -c 'import __graft_entry__ as g; g.build()'`")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _EXPORTS.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


# Status codes whose variant carries four fields (a, b, c, d).
_FOUR_FIELD_CODES = frozenset({84})


def exported_names():
    return list(_EXPORTS)


def status_name(code: int) -> str:
    return lib().sgl_kv_status_name(code).decode()


def _raise(code: int):
    d = _ErrorDetail()
    lib().sgl_kv_last_error(ctypes.byref(d))
    fields = (d.a, d.b, d.c) + ((d.d,) if code in _FOUR_FIELD_CODES else ())
    raise KvError(code, status_name(code), d.name.decode(), fields, d.message.decode())


def _call(fn, *args):
    code = fn(*args)
    if code != OK:
        _raise(code)


def _u64_array(values) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(values, dtype=np.uint64))


def _pu64(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(_u64))


# --- group 1: layout and plan ----------------------------------------------------------------

@dataclass
class KvCacheRuntimeLayout:
    dtype: str
    page_size: int
    num_layers: int
    kv_heads: int
    head_dim: int
    kv_tensors_per_token: int
    bytes_per_token: int
    page_size_bytes: int

    def _c(self) -> _RuntimeLayout:
        return _RuntimeLayout(DTYPES[self.dtype], 0, self.page_size, self.num_layers,
                              self.kv_heads, self.head_dim, self.kv_tensors_per_token,
                              self.bytes_per_token, self.page_size_bytes)

    @classmethod
    def for_model(cls, dtype: str, page_size: int, num_layers: int, kv_heads: int, head_dim: int,
                  kv_tensors_per_token: int = 2) -> "KvCacheRuntimeLayout":
        """Uniform K/V geometry (KvCacheModelLayout::multi_tensor)."""
        elt = lib().sgl_kv_dtype_bytes_per_element(DTYPES[dtype])
        bpt = num_layers * kv_tensors_per_token * kv_heads * head_dim * elt
        return cls(dtype, page_size, num_layers, kv_heads, head_dim, kv_tensors_per_token, bpt,
                   bpt * page_size)


class KvCacheModelLayout:
    """KvCacheModelLayout (kv_cache.rs:68-225): a model's KV geometry before
    the dtype and page size are chosen."""

    def __init__(self, c: _ModelLayout):
        self._c = c

    @classmethod
    def _build(cls, fn, *args) -> "KvCacheModelLayout":
        out = _ModelLayout()
        _call(fn, *args, ctypes.byref(out))
        return cls(out)

    @classmethod
    def multi_tensor(cls, num_layers: int, kv_heads: int, head_dim: int, kv_tensors_per_token: int):
        return cls._build(lib().sgl_kv_model_layout_multi_tensor, num_layers, kv_heads, head_dim,
                          kv_tensors_per_token)

    @classmethod
    def tensor_pair(cls, num_layers: int, key_heads: int, key_head_dim: int, value_heads: int,
                    value_head_dim: int):
        return cls._build(lib().sgl_kv_model_layout_tensor_pair, num_layers, key_heads, key_head_dim,
                          value_heads, value_head_dim)

    @classmethod
    def packed_bytes_per_layer(cls, num_layers: int, bytes_per_token_per_layer: int):
        return cls._build(lib().sgl_kv_model_layout_packed_bytes_per_layer, num_layers,
                          bytes_per_token_per_layer)

    @classmethod
    def packed_mla(cls, num_layers: int, qk_nope_head_dim: int, qk_rope_head_dim: int):
        return cls._build(lib().sgl_kv_model_layout_packed_mla, num_layers, qk_nope_head_dim,
                          qk_rope_head_dim)

    num_layers = property(lambda self: self._c.num_layers)
    kv_heads = property(lambda self: self._c.kv_heads)
    head_dim = property(lambda self: self._c.head_dim)
    kv_tensors_per_token = property(lambda self: self._c.kv_tensors_per_token)

    @property
    def bytes_per_token_per_layer(self):
        return self._c.bytes_per_token_per_layer or None

    def elements_per_token(self):
        out, has = _u64(), ctypes.c_uint32()
        _call(lib().sgl_kv_model_layout_elements_per_token, ctypes.byref(self._c), ctypes.byref(out),
              ctypes.byref(has))
        return out.value if has.value else None

    def token_size_bytes(self, dtype: str) -> int:
        out = _u64()
        _call(lib().sgl_kv_model_layout_token_size_bytes, ctypes.byref(self._c), DTYPES[dtype],
              ctypes.byref(out))
        return out.value

    def tensor_pair_size_bytes(self, dtype: str):
        out, is_pair = (_u64 * 2)(), ctypes.c_uint32()
        _call(lib().sgl_kv_model_layout_tensor_pair_size_bytes, ctypes.byref(self._c), DTYPES[dtype], out,
              ctypes.byref(is_pair))
        return [out[0], out[1]] if is_pair.value else None


class PagedKvCacheLayout:
    """PagedKvCacheLayout (kv_cache.rs:436-823): page -> layer -> tensor -> token."""

    def __init__(self, c: _PagedLayout):
        self._c = c

    @classmethod
    def new(cls, runtime: KvCacheRuntimeLayout, page_count: int) -> "PagedKvCacheLayout":
        out = _PagedLayout()
        rt = runtime._c()
        _call(lib().sgl_kv_paged_layout_new, ctypes.byref(rt), page_count, ctypes.byref(out))
        return cls(out)

    @classmethod
    def for_model(cls, model: KvCacheModelLayout, dtype: str, page_size: int,
                  slot_capacity: int) -> "PagedKvCacheLayout":
        """paged_kv_cache_layout_for_model (backend_model.rs:348-382)."""
        out = _PagedLayout()
        _call(lib().sgl_kv_paged_layout_for_model, ctypes.byref(model._c), DTYPES[dtype], page_size,
              slot_capacity, ctypes.byref(out))
        return cls(out)

    @property
    def runtime(self) -> "KvCacheRuntimeLayout":
        r = self._c.runtime
        name = {v: k for k, v in DTYPES.items()}[r.dtype]
        return KvCacheRuntimeLayout(name, r.page_size, r.num_layers, r.kv_heads, r.head_dim,
                                    r.kv_tensors_per_token, r.bytes_per_token, r.page_size_bytes)

    @classmethod
    def new_with_tensor_pair(cls, runtime: KvCacheRuntimeLayout, page_count: int,
                             key_token_bytes: int, value_token_bytes: int) -> "PagedKvCacheLayout":
        out = _PagedLayout()
        rt = runtime._c()
        _call(lib().sgl_kv_paged_layout_new_with_tensor_pair, ctypes.byref(rt), page_count,
              key_token_bytes, value_token_bytes, ctypes.byref(out))
        return cls(out)

    page_count = property(lambda self: self._c.page_count)
    total_byte_len = property(lambda self: self._c.total_byte_len)
    slot_count = property(lambda self: self._c.slot_count)
    bytes_per_token_per_layer = property(lambda self: self._c.bytes_per_token_per_layer)
    bytes_per_layer_page = property(lambda self: self._c.bytes_per_layer_page)

    @property
    def bytes_per_token_per_tensor(self):
        return None if self._c.tensor_pair else self._c.token_bytes[0]

    def tensor_token_bytes(self, tensor: int) -> int:
        """Bytes of one token of `tensor` in one layer (per-tensor width of a pair layout)."""
        return self._c.token_bytes[min(tensor, 1)]

    @property
    def bytes_per_tensor_page(self):
        return None if self._c.tensor_pair else self._c.tensor_page_bytes

    def _range(self, fn, *args):
        s, e = _u64(), _u64()
        _call(fn, ctypes.byref(self._c), *args, ctypes.byref(s), ctypes.byref(e))
        return (s.value, e.value)

    def page_byte_range(self, page):
        return self._range(lib().sgl_kv_paged_layout_page_byte_range, page)

    def tensor_token_byte_range(self, page, layer, tensor, token):
        return self._range(lib().sgl_kv_paged_layout_tensor_token_byte_range, page, layer, tensor,
                           token)

    def tensor_slot_byte_range(self, layer, tensor, slot):
        return self._range(lib().sgl_kv_paged_layout_tensor_slot_byte_range, layer, tensor, slot)

    def validate_slot_indices(self, slots):
        a = _u64_array(slots)
        _call(lib().sgl_kv_paged_layout_validate_slot_indices, ctypes.byref(self._c), _pu64(a),
              len(a))

    def kv_pair_copy_geometry(self, layer) -> "KvPairCopyLayout":
        out = _PairCopyLayout()
        _call(lib().sgl_kv_paged_layout_kv_pair_copy_geometry, ctypes.byref(self._c), layer,
              ctypes.byref(out))
        return KvPairCopyLayout(out.page_size, out.page_stride_bytes, out.key_in_page_offset,
                                out.value_in_page_offset, out.row_bytes)

    def pool_view(self, base: int, byte_len: int, layer: int, head_layout: int = NHD,
                  heads: int = 1, first_tensor: int = 0, tensor_count: int | None = None,
                  scale: int | None = None) -> PoolView:
        if tensor_count is None:
            tensor_count = min(2, self._c.runtime.kv_tensors_per_token - first_tensor)
        v = PoolView()
        _call(lib().sgl_kv_pool_view_for_layer, ctypes.byref(self._c), base, byte_len,
              head_layout, heads, layer, first_tensor, tensor_count, ctypes.byref(v))
        v.scale = scale
        return v


@dataclass(frozen=True)
class KvPairCopyLayout:
    page_size: int
    page_stride_bytes: int
    key_in_page_offset: int
    value_in_page_offset: int
    row_bytes: int

    def _c(self):
        return _PairCopyLayout(self.page_size, self.page_stride_bytes, self.key_in_page_offset,
                               self.value_in_page_offset, self.row_bytes)


class KvPairCopyPlan:
    """CudaKvPairCopyPlan (cuda_kv_kernels.rs:153-264)."""

    def __init__(self, c: _PairCopyPlan):
        self._c = c

    @classmethod
    def new(cls, row_count, slot_count, layout: KvPairCopyLayout, key_row_stride_bytes,
            value_row_stride_bytes) -> "KvPairCopyPlan":
        out = _PairCopyPlan()
        lay = layout._c()
        _call(lib().sgl_kv_pair_copy_plan_new, row_count, slot_count, ctypes.byref(lay),
              key_row_stride_bytes, value_row_stride_bytes, ctypes.byref(out))
        return cls(out)

    row_count = property(lambda self: self._c.row_count)
    slot_count = property(lambda self: self._c.slot_count)
    key_row_stride_bytes = property(lambda self: self._c.key_row_stride_bytes)
    value_row_stride_bytes = property(lambda self: self._c.value_row_stride_bytes)
    key_rows_required_bytes = property(lambda self: self._c.key_rows_required_bytes)
    value_rows_required_bytes = property(lambda self: self._c.value_rows_required_bytes)
    slot_indices_required_bytes = property(lambda self: self._c.slot_indices_required_bytes)
    pool_required_bytes = property(lambda self: self._c.pool_required_bytes)

    @property
    def layout(self) -> KvPairCopyLayout:
        lay = self._c.layout
        return KvPairCopyLayout(lay.page_size, lay.page_stride_bytes, lay.key_in_page_offset,
                                lay.value_in_page_offset, lay.row_bytes)


def transfer_page_indices(request_index: int, token_offset: int, cache_slots, page_size: int):
    """transfer_page_indices (transfer.rs:679-720): page index of each page-sized
    run of a request's cache slots."""
    a = _u64_array(cache_slots)
    out = np.zeros(max(1, -(-len(a) // max(page_size, 1))), dtype=np.uint64)
    n = _u64()
    _call(lib().sgl_kv_transfer_page_indices, request_index, token_offset, _pu64(a), len(a),
          page_size, _pu64(out), ctypes.byref(n))
    return out[: n.value].tolist()


def build_page_requests(source_base_addr: int, page_size_bytes: int, target_base_offset: int,
                        token_offset: int, token_count: int, page_size: int, page_indices):
    """build_mooncake_kv_transfer_requests (transfer.rs:1945-1997): one page
    write per source page; returns a PAGE_REQUEST_DTYPE array."""
    pages = _u64_array(page_indices)
    out = np.zeros(max(1, len(pages)), dtype=PAGE_REQUEST_DTYPE)
    n = _u64()
    _call(lib().sgl_kv_build_page_requests, source_base_addr, page_size_bytes, target_base_offset,
          token_offset, token_count, page_size, _pu64(pages), len(pages), out.ctypes.data, len(out),
          ctypes.byref(n))
    return out[: n.value]


def build_remote_page_requests(source_base_addr: int, page_size_bytes: int, token_count: int,
                               page_size: int, page_indices, dst_kv_ptrs, dst_kv_indices,
                               dst_kv_item_len: int):
    """build_mooncake_remote_kv_transfer_requests (transfer.rs:1999-2090): every
    source page split into len(dst_kv_ptrs) writes of dst_kv_item_len bytes."""
    pages, ptrs = _u64_array(page_indices), _u64_array(dst_kv_ptrs)
    idx = np.ascontiguousarray(np.asarray(dst_kv_indices, dtype=np.int32))
    out = np.zeros(max(1, len(pages) * max(1, len(ptrs))), dtype=PAGE_REQUEST_DTYPE)
    n = _u64()
    _call(lib().sgl_kv_build_remote_page_requests, source_base_addr, page_size_bytes, token_count,
          page_size, _pu64(pages), len(pages), _pu64(ptrs), len(ptrs),
          idx.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), len(idx), dst_kv_item_len,
          out.ctypes.data, len(out), ctypes.byref(n))
    return out[: n.value]


class CachePageAllocator:
    """CachePageAllocator (crates/sglang-srt/src/cache.rs:340-473)."""

    def __init__(self, slot_capacity: int, page_size: int = 1):
        h = ctypes.c_void_p()
        _call(lib().sgl_kv_page_allocator_new, slot_capacity, page_size, ctypes.byref(h))
        self._h = h.value

    with_page_size = classmethod(lambda cls, slot_capacity, page_size: cls(slot_capacity, page_size))

    def available_pages(self) -> int:
        return lib().sgl_kv_page_allocator_available_pages(self._h)

    def available_slots(self) -> int:
        return lib().sgl_kv_page_allocator_available_slots(self._h)

    def allocate_for_sequence(self, sequence_slots, slot_count: int):
        seq = _u64_array(sequence_slots)
        out = np.zeros(max(1, slot_count), dtype=np.uint64)
        _call(lib().sgl_kv_page_allocator_allocate_for_sequence, self._h, _pu64(seq), len(seq),
              slot_count, _pu64(out))
        return out[:slot_count].tolist()

    def allocate(self, slot_count: int):
        return self.allocate_for_sequence([], slot_count)

    def release(self, cache_pages):
        a = _u64_array(cache_pages)
        _call(lib().sgl_kv_page_allocator_release, self._h, _pu64(a), len(a))

    def reset(self):
        _call(lib().sgl_kv_page_allocator_reset, self._h)

    def __del__(self):
        try:
            if self._h:
                lib().sgl_kv_page_allocator_destroy(self._h)
                self._h = None
        except Exception:
            pass


@dataclass
class PrefixMatch:
    """PrefixMatch (cache.rs:31-36)."""
    matched_token_count: int
    cache_pages: list
    remaining_input_ids: list


def _u32_array(values) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(values, dtype=np.uint32))


class RadixCache:
    """RadixCache (crates/sglang-srt/src/cache.rs:475-547): token ids -> KV
    slots of a cached prompt prefix."""

    def __init__(self):
        h = ctypes.c_void_p()
        _call(lib().sgl_kv_radix_cache_new, ctypes.byref(h))
        self._h = h.value

    def clear(self):
        _call(lib().sgl_kv_radix_cache_clear, self._h)

    def insert(self, input_ids, cache_pages):
        ids, pages = _u32_array(input_ids), _u64_array(cache_pages)
        _call(lib().sgl_kv_radix_cache_insert, self._h,
              ids.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), len(ids), _pu64(pages), len(pages))

    def match_prefix_page_aligned(self, input_ids, page_size: int) -> PrefixMatch:
        ids = _u32_array(input_ids)
        out = np.zeros(max(1, len(ids)), dtype=np.uint64)
        m = _u64()
        _call(lib().sgl_kv_radix_cache_match_prefix, self._h,
              ids.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), len(ids), page_size, ctypes.byref(m),
              _pu64(out))
        n = m.value
        return PrefixMatch(n, out[:n].tolist(), ids[n:].tolist())

    def match_prefix(self, input_ids) -> PrefixMatch:
        return self.match_prefix_page_aligned(input_ids, 1)

    def __del__(self):
        try:
            if self._h:
                lib().sgl_kv_radix_cache_destroy(self._h)
                self._h = None
        except Exception:
            pass


@dataclass
class PlanSpan:
    """One span of KvCacheTransferPlan (transfer.rs:495-505) by request index."""
    request_index: int
    token_offset: int
    token_count: int
    cache_pages: list
    page_indices: list


def transfer_plan_from_prefill_batch(input_token_counts, cached_token_counts, has_disaggregated_params,
                                     out_cache_pages, page_size: int = 1,
                                     forward_mode: int = FORWARD_PREFILL) -> list:
    """KvCacheTransferPlan::from_prefill_worker_batch_with_page_size
    (transfer.rs:604-668) over a prefill batch's per-request token counts,
    PD flags and concatenated cache slots: the spans, in batch order."""
    inp, cached = _u64_array(input_token_counts), _u64_array(cached_token_counts)
    pd = np.ascontiguousarray(np.asarray(has_disaggregated_params, dtype=np.uint8))
    pages = _u64_array(out_cache_pages)
    b = _PrefillBatch(forward_mode, len(inp), _pu64(inp), _pu64(cached),
                      pd.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), _pu64(pages), len(pages))
    spans = np.zeros(max(1, len(inp)), dtype=PLAN_SPAN_DTYPE)
    idx = np.zeros(max(1, len(pages) // max(page_size, 1) + len(inp)), dtype=np.uint64)
    ns, ni = _u64(), _u64()
    _call(lib().sgl_kv_transfer_plan_from_prefill_batch, ctypes.byref(b), page_size, spans.ctypes.data,
          len(spans), _pu64(idx), len(idx), ctypes.byref(ns), ctypes.byref(ni))
    out = []
    for sp in spans[: ns.value]:
        c0, p0 = int(sp["cache_page_offset"]), int(sp["page_index_offset"])
        out.append(PlanSpan(int(sp["request_index"]), int(sp["token_offset"]), int(sp["token_count"]),
                            pages[c0:c0 + int(sp["token_count"])].tolist(),
                            idx[p0:p0 + int(sp["page_index_count"])].tolist()))
    return out


def transfer_span_checksum(request_id: str, bootstrap_host: str, bootstrap_port: int,
                           bootstrap_room: int, data_parallel_rank: int, token_offset: int,
                           token_count: int, page_size: int, cache_pages, page_indices) -> str:
    """KvCacheTransferSpan::descriptor_checksum (transfer.rs:548-570)."""
    rid, host = request_id.encode(), bootstrap_host.encode()
    cp, pi = _u64_array(cache_pages), _u64_array(page_indices)
    out = ctypes.create_string_buffer(65)
    _call(lib().sgl_kv_transfer_span_checksum, rid, len(rid), host, len(host), bootstrap_port,
          bootstrap_room, data_parallel_rank, token_offset, token_count, page_size, _pu64(cp),
          len(cp), _pu64(pi), len(pi), out)
    return out.value.decode()


def sha256_hex(data: bytes) -> str:
    out = ctypes.create_string_buffer(65)
    _call(lib().sgl_kv_sha256_hex, data, len(data), out)
    return out.value.decode()


# --- group 2: device calls -------------------------------------------------------------------

def device_buffer(ptr: int, byte_len: int) -> _DeviceBuffer:
    return _DeviceBuffer(ptr, byte_len)


def rows_view(planes, plane_bytes, row_stride, scale: int | None = None) -> RowsView:
    planes, plane_bytes, row_stride = list(planes), list(plane_bytes), list(row_stride)
    while len(planes) < 2:
        planes.append(None)
        plane_bytes.append(0)
        row_stride.append(0)
    v = RowsView()
    v.planes[0], v.planes[1] = planes[0], planes[1]
    v.plane_bytes[0], v.plane_bytes[1] = plane_bytes
    v.row_stride[0], v.row_stride[1] = row_stride
    v.scale = scale
    return v


def pool_view(base: int, byte_len: int, *, page_size: int, page_stride_bytes: int,
              page_count: int, tensor_offset, row_bytes: int, tensor_count: int, heads: int = 1,
              head_layout: int = NHD, scale: int | None = None,
              value_row_bytes: int = 0) -> PoolView:
    """A pool view filled directly (for pools this library did not describe);
    value_row_bytes gives tensor 1's width when it differs from row_bytes."""
    v = PoolView()
    v.value_row_bytes = value_row_bytes
    v.base, v.byte_len, v.page_size = base, byte_len, page_size
    v.page_stride_bytes, v.page_count = page_stride_bytes, page_count
    offs = list(tensor_offset) + [0, 0]
    v.tensor_offset[0], v.tensor_offset[1] = offs[0], offs[1]
    v.row_bytes, v.tensor_count, v.heads, v.head_layout = row_bytes, tensor_count, heads, head_layout
    v.scale = scale
    return v


def _stream(stream) -> int | None:
    if stream is None:
        return None
    return getattr(stream, "handle", stream)


class RocmKvPairCopyKernels:
    """CudaKvPairCopyKernels (cuda_kv_kernels.rs:416-642) on MI355X, plus the
    per-layer PD transfer calls. ``RocmKvPairCopyKernels.compile(device)``
    loads the prebuilt gfx950 code object (no runtime compilation)."""

    def __init__(self, device: int = 0, code_object: str | None = None):
        if code_object is None and not os.path.exists(CODE_OBJECT_PATH):
            raise ExtensionMissing(f"{CODE_OBJECT_PATH} is not built")
        h = ctypes.c_void_p()
        _call(lib().sgl_rocm_kv_init, device,
              code_object.encode() if code_object else None, ctypes.byref(h))
        self._h = h.value

    compile = classmethod(lambda cls, device=0, code_object=None: cls(device, code_object))

    @property
    def device(self) -> int:
        return lib().sgl_rocm_kv_device(self._h)

    @property
    def cu_count(self) -> int:
        return lib().sgl_rocm_kv_cu_count(self._h)

    def memory_info(self):
        """CudaContext::memory_info (crates/sglang-kernel/src/cuda.rs:496-511):
        (free_bytes, total_bytes) of the device."""
        f, t = _u64(), _u64()
        _call(lib().sgl_rocm_kv_memory_info, self._h, ctypes.byref(f), ctypes.byref(t))
        return f.value, t.value

    def close(self):
        if self._h:
            _call(lib().sgl_rocm_kv_destroy, self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @staticmethod
    def _buffers(keys, keys_offset, values, values_offset, slot_indices, slot_indices_offset,
                 pool, pool_offset) -> _PairCopyBuffers:
        def db(b):
            return _DeviceBuffer(b.ptr, b.nbytes) if hasattr(b, "nbytes") else b
        return _PairCopyBuffers(db(keys), keys_offset, db(values), values_offset,
                                db(slot_indices), slot_indices_offset, db(pool), pool_offset)

    def scatter(self, plan: KvPairCopyPlan, *, keys, values, slot_indices, pool, keys_offset=0,
                values_offset=0, slot_indices_offset=0, pool_offset=0, stream=None):
        """CudaKvPairCopyKernels::scatter: strided K/V rows -> pool slots; synchronous."""
        b = self._buffers(keys, keys_offset, values, values_offset, slot_indices,
                          slot_indices_offset, pool, pool_offset)
        _call(lib().sgl_rocm_kv_pair_scatter, self._h, ctypes.byref(plan._c), ctypes.byref(b),
              _stream(stream))

    def gather(self, plan: KvPairCopyPlan, *, pool, slot_indices, keys, values, pool_offset=0,
               slot_indices_offset=0, keys_offset=0, values_offset=0, stream=None):
        """CudaKvPairCopyKernels::gather: pool slots -> strided K/V rows; synchronous."""
        b = self._buffers(keys, keys_offset, values, values_offset, slot_indices,
                          slot_indices_offset, pool, pool_offset)
        _call(lib().sgl_rocm_kv_pair_gather, self._h, ctypes.byref(plan._c), ctypes.byref(b),
              _stream(stream))

    def pack_layer(self, src: PoolView, slots: _DeviceBuffer, row_count: int, dst: RowsView,
                   stream=None):
        _call(lib().sgl_rocm_kv_pack_layer, self._h, ctypes.byref(src), ctypes.byref(slots),
              row_count, ctypes.byref(dst), _stream(stream))

    def unpack_layer(self, src: RowsView, row_count: int, dst: PoolView, slots: _DeviceBuffer,
                     stream=None):
        _call(lib().sgl_rocm_kv_unpack_layer, self._h, ctypes.byref(src), row_count,
              ctypes.byref(dst), ctypes.byref(slots), _stream(stream))

    def pack_layers(self, src: PoolView, pool_layer_stride: int, layer_count: int,
                    slots: _DeviceBuffer, row_count: int, dst: RowsView, rows_layer_stride: int,
                    stream=None):
        """Pack `layer_count` consecutive layers in one launch."""
        _call(lib().sgl_rocm_kv_pack_layers, self._h, ctypes.byref(src), pool_layer_stride,
              layer_count, ctypes.byref(slots), row_count, ctypes.byref(dst), rows_layer_stride,
              _stream(stream))

    def unpack_layers(self, src: RowsView, rows_layer_stride: int, layer_count: int,
                      row_count: int, dst: PoolView, pool_layer_stride: int, slots: _DeviceBuffer,
                      stream=None):
        """Unpack `layer_count` consecutive layers in one launch."""
        _call(lib().sgl_rocm_kv_unpack_layers, self._h, ctypes.byref(src), rows_layer_stride,
              layer_count, row_count, ctypes.byref(dst), pool_layer_stride, ctypes.byref(slots),
              _stream(stream))

    def write_tensor_slots(self, layout: "PagedKvCacheLayout", pool: _DeviceBuffer, layer: int,
                           tensor: int, slots: _DeviceBuffer, count: int, source: _DeviceBuffer,
                           source_offset: int = 0, source_row_stride: int | None = None,
                           stream=None):
        """Batched CudaKvStorage::write_tensor_slot_from_device: rows
        source_offset + i * stride -> (layer, tensor, slots[i]) of the pool.
        The stride defaults to the tensor's token width."""
        if source_row_stride is None:
            source_row_stride = layout.tensor_token_bytes(tensor)
        _call(lib().sgl_rocm_kv_write_tensor_slots, self._h, ctypes.byref(layout._c),
              ctypes.byref(pool), layer, tensor, ctypes.byref(slots), count, ctypes.byref(source),
              source_offset, source_row_stride, _stream(stream))

    def write_tensor_pair_slots(self, layout: "PagedKvCacheLayout", pool: _DeviceBuffer, layer: int,
                                slots: _DeviceBuffer, count: int, keys: _DeviceBuffer, values: _DeviceBuffer,
                                keys_offset: int = 0, keys_row_stride: int | None = None,
                                values_offset: int = 0, values_row_stride: int | None = None, stream=None):
        """Both tensors of `layer` for `count` slots in one launch: key rows
        keys_offset + i * stride and value rows values_offset + i * stride
        (strides default to each tensor's token width)."""
        if keys_row_stride is None:
            keys_row_stride = layout.tensor_token_bytes(0)
        if values_row_stride is None:
            values_row_stride = layout.tensor_token_bytes(1)
        _call(lib().sgl_rocm_kv_write_tensor_pair_slots, self._h, ctypes.byref(layout._c),
              ctypes.byref(pool), layer, ctypes.byref(slots), count, ctypes.byref(keys), keys_offset,
              keys_row_stride, ctypes.byref(values), values_offset, values_row_stride, _stream(stream))

    def read_tensor_slots(self, layout: "PagedKvCacheLayout", pool: _DeviceBuffer, layer: int,
                          tensor: int, slots: _DeviceBuffer, count: int, destination: _DeviceBuffer,
                          destination_offset: int = 0, destination_row_stride: int | None = None,
                          stream=None):
        """Batched CudaKvStorage::read_tensor_slot_to_device."""
        if destination_row_stride is None:
            destination_row_stride = layout.tensor_token_bytes(tensor)
        _call(lib().sgl_rocm_kv_read_tensor_slots, self._h, ctypes.byref(layout._c),
              ctypes.byref(pool), layer, tensor, ctypes.byref(slots), count,
              ctypes.byref(destination), destination_offset, destination_row_stride,
              _stream(stream))

    def transfer_layer(self, src: PoolView, src_slots: _DeviceBuffer, row_count: int,
                       dst: PoolView, dst_slots: _DeviceBuffer, stream=None):
        _call(lib().sgl_rocm_kv_transfer_layer, self._h, ctypes.byref(src),
              ctypes.byref(src_slots), row_count, ctypes.byref(dst), ctypes.byref(dst_slots),
              _stream(stream))

    def transfer_layers(self, src: PoolView, src_layer_stride: int, layer_count: int,
                        src_slots: _DeviceBuffer, row_count: int, dst: PoolView,
                        dst_layer_stride: int, dst_slots: _DeviceBuffer, stream=None):
        """Pool -> pool over `layer_count` consecutive layers in one launch."""
        _call(lib().sgl_rocm_kv_transfer_layers, self._h, ctypes.byref(src), src_layer_stride,
              layer_count, ctypes.byref(src_slots), row_count, ctypes.byref(dst), dst_layer_stride,
              ctypes.byref(dst_slots), _stream(stream))

    def resolve_spans(self, page_size: int, page_count: int, spans: _DeviceBuffer,
                      span_count: int, page_table: _DeviceBuffer, page_table_len: int,
                      row_count: int, out_slots: _DeviceBuffer, stream=None):
        _call(lib().sgl_rocm_kv_resolve_spans, self._h, page_size, page_count,
              ctypes.byref(spans), span_count, ctypes.byref(page_table), page_table_len,
              row_count, ctypes.byref(out_slots), _stream(stream))

    def execute_page_requests(self, requests: _DeviceBuffer, count: int, max_length: int,
                              source_region: _DeviceBuffer, target_region: _DeviceBuffer,
                              offsets_are_addresses: bool = False, stream=None):
        """Page requests (PAGE_REQUEST_DTYPE, on the device) as device copies."""
        _call(lib().sgl_rocm_kv_execute_page_requests, self._h, ctypes.byref(requests), count,
              max_length, ctypes.byref(source_region), ctypes.byref(target_region),
              int(offsets_are_addresses), _stream(stream))

    def paged_attention(self, plan: "PagedAttentionPlan", *, max_sequence_length: int = 0,
                        stream=None, **buffers):
        """CudaBf16PagedAttentionKernels::forward (cuda_attention.rs:681-850):
        keyword buffers queries, query_request_indices, query_sequence_lengths,
        request_slot_offsets, sequence_slots, pool and output (objects with
        .ptr/.nbytes, or device_buffer(...)), each with an optional
        <name>_offset. Synchronous; bad metadata raises DeviceMetadataInvalid."""
        _paged_attention(lib().sgl_rocm_kv_paged_attention, self, plan, buffers,
                         max_sequence_length, stream)

    def paged_attention_async(self, plan: "PagedAttentionPlan", *, max_sequence_length: int = 0,
                              stream=None, **buffers):
        """paged_attention without the wait: bad metadata surfaces at the next
        check_errors. Buffers as for paged_attention."""
        _paged_attention(lib().sgl_rocm_kv_paged_attention_async, self, plan, buffers,
                         max_sequence_length, stream)

    def paged_attention_async_noalloc(self, plan: "PagedAttentionPlan", *, max_sequence_length: int = 0,
                                      stream=None, **buffers):
        """paged_attention_async with the split records in the library's
        static device workspace (NOALLOC_WORKSPACE_BYTES per device): no
        device allocation; launches needing more are refused."""
        _paged_attention(lib().sgl_rocm_kv_paged_attention_async_noalloc, self, plan, buffers,
                         max_sequence_length, stream)

    def check_errors(self, stream=None):
        _call(lib().sgl_rocm_kv_check_errors, self._h, _stream(stream))

    def fill_synthetic(self, buffer: _DeviceBuffer, seed: int, kind: int = FILL_BITS, stream=None):
        _call(lib().sgl_rocm_kv_fill_synthetic, self._h, ctypes.byref(buffer), seed, kind,
              _stream(stream))

    def stream_ceiling(self, kind: int, src, dst, nbytes: int, stream=None):
        """The device's streaming ceilings (STREAM_COPY / READ / WRITE of
        `nbytes` contiguous bytes); src or dst may be None where unused."""
        s = src if src is not None else _DeviceBuffer(None, 0)
        d = dst if dst is not None else _DeviceBuffer(None, 0)
        _call(lib().sgl_rocm_kv_stream, self._h, kind, ctypes.byref(s), ctypes.byref(d), nbytes,
              _stream(stream))


class LayerPipeline:
    """sgl_rocm_kv_pipeline: a whole-request transfer, layer by layer, with
    pack, the optional pinned-host hop (D2H then H2D) and unpack overlapped
    across layers on four streams. ``send``/``recv`` are pairs of device
    buffers and ``host`` a pair of pinned host buffers (objects with .ptr and
    .nbytes), each holding one layer's rows."""

    def __init__(self, kernels: "RocmKvPairCopyKernels", src_layers, dst_layers, src_slots,
                 dst_slots, row_count: int, send, recv=None, host=None):
        n = len(src_layers)
        self._src = (PoolView * n)(*src_layers)
        self._dst = (PoolView * n)(*dst_layers)
        d = _PipelineDesc()
        d.layers, d.staged = n, int(host is not None)
        d.src_layers, d.dst_layers = self._src, self._dst
        d.src_slots, d.dst_slots, d.row_count = src_slots, dst_slots, row_count
        for i in range(2):
            d.send[i] = _DeviceBuffer(send[i].ptr, send[i].nbytes)
            if host is not None:
                d.recv[i] = _DeviceBuffer(recv[i].ptr, recv[i].nbytes)
                d.host[i] = host[i].ptr
        d.host_bytes = min(h.nbytes for h in host) if host is not None else 0
        self.layers = n
        h = ctypes.c_void_p()
        _call(lib().sgl_rocm_kv_pipeline_create, kernels._h, ctypes.byref(d), ctypes.byref(h))
        self._h = h.value

    def run(self, after=None):
        _call(lib().sgl_rocm_kv_pipeline_run, self._h, getattr(after, "handle", after))

    def wait(self):
        _call(lib().sgl_rocm_kv_pipeline_wait, self._h)

    def layer_times(self, layer: int):
        """(pack, d2h, h2d, unpack, latency) in ms of `layer`'s last run."""
        ms = (ctypes.c_float * 5)()
        _call(lib().sgl_rocm_kv_pipeline_layer_times, self._h, layer, ms)
        return tuple(ms)

    def elapsed_ms(self) -> float:
        ms = ctypes.c_float()
        _call(lib().sgl_rocm_kv_pipeline_elapsed, self._h, ctypes.byref(ms))
        return ms.value

    def close(self):
        if self._h:
            _call(lib().sgl_rocm_kv_pipeline_destroy, self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


BACKEND_DIRECT, BACKEND_STAGED = 0, 1
NOALLOC_WORKSPACE_BYTES = 128 << 20   # SGL_KV_NOALLOC_WORKSPACE_BYTES
TRANSFER_COMPLETED, TRANSFER_FAILED, TRANSFER_CANCELED = 0, 1, 2


@dataclass(frozen=True)
class KvTransferCompletionEvent:
    """KvTransferCompletionEvent (transfer.rs:1073-1078); error_code is the
    device error's status for a FAILED event."""
    bootstrap_room: int
    descriptor_checksum: str
    status: int
    error_code: int = 0


class RocmKvTransferBackend:
    """sgl_rocm_kv_backend: KvTransferBackend (transfer.rs:1145-1151) over a
    prefill pool and a decode pool on one device. ``mode`` is BACKEND_DIRECT
    (one pool-to-pool launch per span) or BACKEND_STAGED (the layer pipeline
    through pinned host memory); ``max_rows`` bounds a span's token_count."""

    def __init__(self, kernels: "RocmKvPairCopyKernels", mode: int = BACKEND_DIRECT,
                 max_rows: int = 1 << 20):
        self._kernels = kernels  # the context must outlive the backend
        cfg = _BackendConfig(mode, 0, max_rows)
        h = ctypes.c_void_p()
        _call(lib().sgl_rocm_kv_backend_create, kernels._h, ctypes.byref(cfg), ctypes.byref(h))
        self._h = h.value

    @staticmethod
    def _memory(layout: PagedKvCacheLayout, base: int, byte_len: int, head_layout: int,
                heads: int) -> _BackendMemory:
        return _BackendMemory(layout._c, base, byte_len, head_layout, 0, heads)

    def register(self, prefill: PagedKvCacheLayout, prefill_base: int, prefill_len: int,
                 decode: PagedKvCacheLayout, decode_base: int, decode_len: int, *,
                 prefill_head_layout: int = NHD, prefill_heads: int = 0,
                 decode_head_layout: int = NHD, decode_heads: int = 0):
        """Registers both pools; heads 0 takes the layout's kv_heads."""
        p = self._memory(prefill, prefill_base, prefill_len, prefill_head_layout, prefill_heads)
        d = self._memory(decode, decode_base, decode_len, decode_head_layout, decode_heads)
        _call(lib().sgl_rocm_kv_backend_register, self._h, ctypes.byref(p), ctypes.byref(d))

    def register_pools(self, prefill: "KvCachePool", decode: "KvCachePool", *,
                       prefill_head_layout: int = NHD, prefill_heads: int = 0,
                       decode_head_layout: int = NHD, decode_heads: int = 0):
        """Registers two storage-backed pools (sgl_rocm_kv_storage_backend_memory)."""
        p = prefill.storage().backend_memory(prefill.layout(), prefill_head_layout, prefill_heads)
        d = decode.storage().backend_memory(decode.layout(), decode_head_layout, decode_heads)
        _call(lib().sgl_rocm_kv_backend_register, self._h, ctypes.byref(p), ctypes.byref(d))

    def submit(self, bootstrap_room: int, descriptor_checksum: str, token_offset: int,
               cache_slots, dst_page_table):
        """Submits one span: prefill `cache_slots` hold the request's tokens
        token_offset.. ; the decode side holds them in `dst_page_table`."""
        slots = _u64_array(cache_slots)
        table = np.ascontiguousarray(np.asarray(dst_page_table, dtype=np.int32))
        d = self._span(bootstrap_room, descriptor_checksum, token_offset, slots)
        d.dst_page_table = table.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))
        d.dst_page_table_len = len(table)
        _call(lib().sgl_rocm_kv_backend_submit, self._h, ctypes.byref(d))

    def submit_device_table(self, bootstrap_room: int, descriptor_checksum: str, token_offset: int,
                            cache_slots, dst_page_table: "_DeviceBuffer", dst_page_table_len: int):
        """As submit, with the decode page table in device memory (int32
        entries): the decode slots are resolved on the device, and a bad entry
        fails the span at poll (DevicePageIndexOutOfRange)."""
        slots = _u64_array(cache_slots)
        d = self._span(bootstrap_room, descriptor_checksum, token_offset, slots)
        d.dst_page_table = ctypes.cast(ctypes.c_void_p(dst_page_table.ptr), ctypes.POINTER(ctypes.c_int32))
        d.dst_page_table_len = dst_page_table_len
        _call(lib().sgl_rocm_kv_backend_submit_device_table, self._h, ctypes.byref(d))

    @staticmethod
    def _span(bootstrap_room: int, descriptor_checksum: str, token_offset: int, slots: np.ndarray):
        d = _SpanDesc()
        d.bootstrap_room = bootstrap_room
        d.descriptor_checksum = descriptor_checksum.encode()[:64]
        d.token_offset, d.token_count = token_offset, len(slots)
        d.cache_slots = slots.ctypes.data_as(ctypes.POINTER(_u64))
        return d

    def poll(self, capacity: int = 256):
        """(events, pending_transfers), as KvTransferPoll (transfer.rs:1122-1143)."""
        events = (_TransferEvent * max(capacity, 1))()
        n, pending = _u64(), _u64()
        _call(lib().sgl_rocm_kv_backend_poll, self._h, events, capacity, ctypes.byref(n),
              ctypes.byref(pending))
        out = [KvTransferCompletionEvent(e.bootstrap_room, e.descriptor_checksum.decode(),
                                         e.status, e.error_code) for e in events[:n.value]]
        return out, pending.value

    def cancel(self, bootstrap_room: int):
        _call(lib().sgl_rocm_kv_backend_cancel, self._h, bootstrap_room)

    def wait(self):
        _call(lib().sgl_rocm_kv_backend_wait, self._h)

    def shutdown(self):
        _call(lib().sgl_rocm_kv_backend_shutdown, self._h)

    def close(self):
        if self._h:
            _call(lib().sgl_rocm_kv_backend_destroy, self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


@dataclass
class TransferableKvCacheRegion:
    """TransferableKvCacheRegion (nexus-transfer, used at cuda_kv_cache.rs:464-468)."""
    base_addr: int
    byte_len: int
    page_size_bytes: int


@dataclass
class MooncakeRemoteKvLayout:
    """MooncakeRemoteKvLayout (crates/sglang-srt/src/transfer.rs:1651-1656)."""
    dst_kv_ptrs: list
    dst_kv_indices: list
    dst_kv_item_len: int


def memory_location_label(kind: int, location_id: int) -> str:
    """mooncake_memory_location_label (transfer.rs:1662-1676): "hip:0" for
    ROCm device 0; Metal, Xpu and Hpu raise UnsupportedMemoryLocation."""
    out = (ctypes.c_char * 32)()
    _call(lib().sgl_kv_memory_location_label, kind, location_id, out)
    return out.value.decode()


class TransferableKvCacheMemory:
    """TransferableKvCacheMemory (nexus-transfer, un-vendored; pinned at
    crates/sglang-srt/Cargo.toml:35): regions, logical page size, location."""

    def __init__(self, regions, page_size_bytes: int, location_kind: int, location_id: int):
        self._regions = [r if isinstance(r, TransferableKvCacheRegion) else TransferableKvCacheRegion(*r)
                         for r in regions]
        self._page_size_bytes = page_size_bytes
        self._location = (location_kind, location_id)

    @classmethod
    def _from_c(cls, c: _TransferableMemory) -> "TransferableKvCacheMemory":
        regions = [TransferableKvCacheRegion(r.base_addr, r.byte_len, r.page_size_bytes)
                   for r in c.regions[: c.region_count]]
        return cls(regions, c.page_size_bytes, c.location_kind, c.location_id)

    def _c(self) -> _TransferableMemory:
        c = _TransferableMemory()
        for i, r in enumerate(self._regions[:MAX_MEMORY_REGIONS]):
            c.regions[i] = _MemoryRegion(r.base_addr, r.byte_len, r.page_size_bytes)
        c.region_count = len(self._regions)
        c.page_size_bytes = self._page_size_bytes
        c.location_kind, c.location_id = self._location
        return c

    def regions(self):
        return list(self._regions)

    def page_size_bytes(self) -> int:
        return self._page_size_bytes

    def location(self):
        """(sgl_kv_memory_location_kind, device id or numa node)."""
        return self._location

    def location_label(self) -> str:
        return memory_location_label(*self._location)

    def mooncake_decode_remote_layout(self, dst_kv_indices) -> MooncakeRemoteKvLayout:
        """mooncake_decode_remote_layout (transfer.rs:1693-1703)."""
        c = self._c()
        ptrs = (_u64 * MAX_MEMORY_REGIONS)()
        n, item = _u64(), _u64()
        _call(lib().sgl_kv_transferable_memory_decode_remote_layout, ctypes.byref(c), ptrs,
              MAX_MEMORY_REGIONS, ctypes.byref(n), ctypes.byref(item))
        return MooncakeRemoteKvLayout(list(ptrs[: n.value]), [int(i) for i in dst_kv_indices], item.value)


@dataclass
class KvCacheTensorLocation:
    """CudaKvCacheTensorLocation (cuda_kv_cache.rs:103-107)."""
    device_ptr: int
    byte_offset: int
    byte_len: int


def _stream_handle(stream):
    return None if stream is None else getattr(stream, "handle", stream)


def _as_db(b) -> _DeviceBuffer:
    return b if isinstance(b, _DeviceBuffer) else _DeviceBuffer(b.ptr, b.nbytes)


class RocmKvSlotMap:
    """CudaKvCacheSlotMap (cuda_kv_cache.rs:109-140): u64 slots on the device
    plus the host slots they were validated with."""

    def __init__(self, handle: int):
        self._h = handle

    def __len__(self) -> int:
        return lib().sgl_rocm_kv_slot_map_len(self._h)

    def slots(self) -> np.ndarray:
        n = len(self)
        ptr = lib().sgl_rocm_kv_slot_map_slots(self._h)
        return np.ctypeslib.as_array(ptr, shape=(n,)).copy() if n else np.zeros(0, np.uint64)

    def allocation(self) -> _DeviceBuffer:
        b = _DeviceBuffer()
        _call(lib().sgl_rocm_kv_slot_map_allocation, self._h, ctypes.byref(b))
        return b

    def close(self):
        if self._h:
            _call(lib().sgl_rocm_kv_slot_map_destroy, self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class RocmKvStorage:
    """CudaKvStorage (cuda_kv_cache.rs:170-509) on MI355X: a library-owned,
    zero-filled device allocation holding a paged pool."""

    def __init__(self, handle: int):
        self._h = handle

    @classmethod
    def allocate(cls, kernels: "RocmKvPairCopyKernels", byte_len: int, page_size_bytes: int) -> "RocmKvStorage":
        """CudaKvStorage::allocate (:177-189)."""
        h = ctypes.c_void_p()
        _call(lib().sgl_rocm_kv_storage_allocate, kernels._h, byte_len, page_size_bytes, ctypes.byref(h))
        return cls(h.value)

    @classmethod
    def allocate_placed(cls, kernels: "RocmKvPairCopyKernels", byte_len: int, page_size_bytes: int,
                        probe_view: "PoolView", probe_rows: _DeviceBuffer | None, candidates: int,
                        stream=None, probe_source: "PoolView | None" = None) -> tuple["RocmKvStorage", dict]:
        """allocate(), keeping the fastest of `candidates` allocations for the
        scatter `probe_view` describes: an unpack from `probe_rows` (scratch),
        or a pool-to-pool transfer from `probe_source` when given (no
        counterpart in the reference). Returns the storage and the probe
        report."""
        h = ctypes.c_void_p()
        r = _PlacementReport()
        _call(lib().sgl_rocm_kv_storage_allocate_placed, kernels._h, byte_len, page_size_bytes,
              ctypes.byref(probe_view), None if probe_rows is None else ctypes.byref(probe_rows),
              None if probe_source is None else ctypes.byref(probe_source), candidates, _stream(stream),
              ctypes.byref(h), ctypes.byref(r))
        report = {"candidates": r.candidates, "chosen": r.chosen, "probe_rows": r.probe_rows,
                  "probe_us": [float(r.probe_us[i]) for i in range(r.candidates)]}
        return cls(h.value), report

    def allocation(self) -> _DeviceBuffer:
        b = _DeviceBuffer()
        _call(lib().sgl_rocm_kv_storage_allocation, self._h, ctypes.byref(b))
        return b

    @property
    def device_ptr(self) -> int:
        return self.allocation().ptr or 0

    def byte_len(self) -> int:
        return lib().sgl_rocm_kv_storage_byte_len(self._h)

    def page_size_bytes(self) -> int:
        return lib().sgl_rocm_kv_storage_page_size_bytes(self._h)

    def device_ordinal(self) -> int:
        return lib().sgl_rocm_kv_storage_device(self._h)

    def clear(self):
        """KvCacheStorage::clear (impl :449-452)."""
        _call(lib().sgl_rocm_kv_storage_clear, self._h)

    def validate_layout(self, layout: "PagedKvCacheLayout"):
        _call(lib().sgl_rocm_kv_storage_validate_layout, self._h, ctypes.byref(layout._c))

    def write_page(self, layout: "PagedKvCacheLayout", page_index: int, data):
        """CudaKvStorage::write_page (:224-239)."""
        a = np.ascontiguousarray(np.frombuffer(bytes(data), dtype=np.uint8)
                                 if isinstance(data, (bytes, bytearray)) else np.asarray(data, dtype=np.uint8))
        _call(lib().sgl_rocm_kv_storage_write_page, self._h, ctypes.byref(layout._c), page_index,
              a.ctypes.data if a.size else None, a.size)

    def read_page(self, layout: "PagedKvCacheLayout", page_index: int, nbytes: int | None = None) -> np.ndarray:
        """CudaKvStorage::read_page (:241-256); nbytes defaults to the page size."""
        n = layout.runtime.page_size_bytes if nbytes is None else nbytes
        out = np.zeros(n, dtype=np.uint8)
        _call(lib().sgl_rocm_kv_storage_read_page, self._h, ctypes.byref(layout._c), page_index,
              out.ctypes.data if n else None, n)
        return out

    def write_tensor_slot_from_device(self, layout: "PagedKvCacheLayout", layer: int, tensor: int, slot: int,
                                      source, source_offset: int = 0, stream=None):
        """CudaKvStorage::write_tensor_slot_from_device (:258-274); asynchronous."""
        src = _as_db(source)
        _call(lib().sgl_rocm_kv_storage_write_tensor_slot, self._h, ctypes.byref(layout._c), layer, tensor, slot,
              ctypes.byref(src), source_offset, _stream_handle(stream))

    def read_tensor_slot_to_device(self, layout: "PagedKvCacheLayout", layer: int, tensor: int, slot: int,
                                   destination, destination_offset: int = 0, stream=None):
        """CudaKvStorage::read_tensor_slot_to_device (:276-294); asynchronous."""
        dst = _as_db(destination)
        _call(lib().sgl_rocm_kv_storage_read_tensor_slot, self._h, ctypes.byref(layout._c), layer, tensor, slot,
              ctypes.byref(dst), destination_offset, _stream_handle(stream))

    def tensor_location(self, layout: "PagedKvCacheLayout", page: int, layer: int, tensor: int,
                        token: int) -> KvCacheTensorLocation:
        out = _TensorLocation()
        _call(lib().sgl_rocm_kv_storage_tensor_location, self._h, ctypes.byref(layout._c), page, layer, tensor,
              token, ctypes.byref(out))
        return KvCacheTensorLocation(out.device_ptr, out.byte_offset, out.byte_len)

    def slot_location(self, layout: "PagedKvCacheLayout", layer: int, tensor: int, slot: int) -> KvCacheTensorLocation:
        """CudaKvStorage::slot_location (:390-403)."""
        out = _TensorLocation()
        _call(lib().sgl_rocm_kv_storage_slot_location, self._h, ctypes.byref(layout._c), layer, tensor, slot,
              ctypes.byref(out))
        return KvCacheTensorLocation(out.device_ptr, out.byte_offset, out.byte_len)

    def upload_slot_map(self, layout: "PagedKvCacheLayout", slots) -> RocmKvSlotMap:
        """CudaKvStorage::upload_slot_map (:199-222)."""
        a = _u64_array(slots)
        h = ctypes.c_void_p()
        _call(lib().sgl_rocm_kv_storage_upload_slot_map, self._h, ctypes.byref(layout._c),
              _pu64(a) if a.size else None, a.size, ctypes.byref(h))
        return RocmKvSlotMap(h.value)

    @staticmethod
    def _rows(keys, key_row_stride_bytes, values, value_row_stride_bytes, keys_offset, values_offset):
        return _SlotRows(_as_db(keys), keys_offset, key_row_stride_bytes, _as_db(values), values_offset,
                         value_row_stride_bytes)

    def write_kv_slots_from_device(self, kernels: "RocmKvPairCopyKernels", layout: "PagedKvCacheLayout",
                                   layer: int, slot_map: RocmKvSlotMap, *, keys, key_row_stride_bytes: int,
                                   values, value_row_stride_bytes: int, keys_offset: int = 0,
                                   values_offset: int = 0, stream=None):
        """CudaKvStorage::write_kv_slots_from_device (:296-334)."""
        r = self._rows(keys, key_row_stride_bytes, values, value_row_stride_bytes, keys_offset, values_offset)
        _call(lib().sgl_rocm_kv_storage_write_kv_slots, kernels._h, self._h, ctypes.byref(layout._c), layer,
              slot_map._h, ctypes.byref(r), _stream_handle(stream))

    def read_kv_slots_to_device(self, kernels: "RocmKvPairCopyKernels", layout: "PagedKvCacheLayout",
                                layer: int, slot_map: RocmKvSlotMap, *, keys, key_row_stride_bytes: int,
                                values, value_row_stride_bytes: int, keys_offset: int = 0,
                                values_offset: int = 0, stream=None):
        """CudaKvStorage::read_kv_slots_to_device (:336-374)."""
        r = self._rows(keys, key_row_stride_bytes, values, value_row_stride_bytes, keys_offset, values_offset)
        _call(lib().sgl_rocm_kv_storage_read_kv_slots, kernels._h, self._h, ctypes.byref(layout._c), layer,
              slot_map._h, ctypes.byref(r), _stream_handle(stream))

    def transferable_kv_cache_memory(self) -> TransferableKvCacheMemory:
        """impl KvCacheMemoryProvider for CudaKvStorage (:455-476), located on
        KvCacheMemoryLocation::Rocm."""
        c = _TransferableMemory()
        _call(lib().sgl_rocm_kv_storage_transferable_memory, self._h, ctypes.byref(c))
        return TransferableKvCacheMemory._from_c(c)

    def backend_memory(self, layout: "PagedKvCacheLayout", head_layout: int = NHD, heads: int = 0):
        m = _BackendMemory()
        _call(lib().sgl_rocm_kv_storage_backend_memory, self._h, ctypes.byref(layout._c), head_layout, heads,
              ctypes.byref(m))
        return m

    def close(self):
        if self._h:
            _call(lib().sgl_rocm_kv_storage_destroy, self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class KvCachePool:
    """KvCachePool<RocmKvStorage> (kv_cache.rs:835-896): a layout and the
    storage it addresses."""

    def __init__(self, layout: "PagedKvCacheLayout", storage: RocmKvStorage):
        self._layout, self._storage = layout, storage

    def layout(self) -> "PagedKvCacheLayout":
        return self._layout

    def storage(self) -> RocmKvStorage:
        return self._storage

    storage_mut = storage

    def clear(self):
        self._storage.clear()

    def transferable_kv_cache_memory(self) -> TransferableKvCacheMemory:
        return self._storage.transferable_kv_cache_memory()

    def close(self):
        self._storage.close()


def allocate_rocm_kv_cache(kernels: "RocmKvPairCopyKernels", runtime: KvCacheRuntimeLayout,
                           page_count: int) -> KvCachePool:
    """allocate_cuda_kv_cache (cuda_kv_cache.rs:478-490) on the kernels' device."""
    out = _PagedLayout()
    h = ctypes.c_void_p()
    _call(lib().sgl_rocm_kv_cache_allocate, kernels._h, ctypes.byref(runtime._c()), page_count,
          ctypes.byref(out), ctypes.byref(h))
    return KvCachePool(PagedKvCacheLayout(out), RocmKvStorage(h.value))


def allocate_rocm_kv_pool(kernels: "RocmKvPairCopyKernels", layout: "PagedKvCacheLayout") -> KvCachePool:
    """A zero-filled storage for an existing layout (a tensor pair included),
    checked as KvCachePool::new does (kv_cache.rs:849-856)."""
    h = ctypes.c_void_p()
    _call(lib().sgl_rocm_kv_pool_allocate, kernels._h, ctypes.byref(layout._c), ctypes.byref(h))
    return KvCachePool(layout, RocmKvStorage(h.value))


class PagedAttentionPlan:
    """CudaBf16PagedAttentionPlan (cuda_attention.rs:239-430), plus the
    head layout of the pages (NHD as the reference, or HND)."""

    def __init__(self, c: _AttentionPlan):
        self._c = c

    @classmethod
    def new(cls, *, query_count: int, request_count: int, sequence_slot_count: int,
            slot_count: int, query_head_count: int, kv_head_count: int, query_key_head_dim: int,
            value_head_dim: int, scale: float, page_size: int, page_stride_bytes: int,
            key_in_page_offset: int, value_in_page_offset: int, key_row_bytes: int,
            value_row_bytes: int, head_layout: int = NHD,
            exact_weights: bool = False, fast_weights: bool = False) -> "PagedAttentionPlan":
        flags = (ATTN_EXACT_WEIGHTS if exact_weights else 0) | (ATTN_FAST_WEIGHTS if fast_weights else 0)
        cfg = _AttentionPlanConfig(query_count, request_count, sequence_slot_count, slot_count,
                                   query_head_count, kv_head_count, query_key_head_dim,
                                   value_head_dim, scale, flags,
                                   _AttentionLayout(page_size, page_stride_bytes,
                                                    key_in_page_offset, value_in_page_offset,
                                                    key_row_bytes, value_row_bytes, head_layout, 0))
        out = _AttentionPlan()
        _call(lib().sgl_kv_attention_plan_new, ctypes.byref(cfg), ctypes.byref(out))
        return cls(out)

    @classmethod
    def for_layer(cls, layout: PagedKvCacheLayout, layer: int, query_count: int,
                  request_count: int, sequence_slot_count: int, query_head_count: int,
                  scale: float, head_layout: int = NHD,
                  exact_weights: bool = False, fast_weights: bool = False) -> "PagedAttentionPlan":
        """CudaBf16PagedAttentionExecutor::plan / build_plan
        (crates/sglang-srt/src/cuda_attention.rs:438-572). `exact_weights` /
        `fast_weights` set ATTN_EXACT_WEIGHTS / ATTN_FAST_WEIGHTS on the plan
        the C entry point returns."""
        out = _AttentionPlan()
        _call(lib().sgl_kv_attention_plan_for_layer, ctypes.byref(layout._c), layer, query_count,
              request_count, sequence_slot_count, query_head_count, scale, head_layout,
              ctypes.byref(out))
        if exact_weights:
            out.config.flags |= ATTN_EXACT_WEIGHTS
        if fast_weights:
            out.config.flags |= ATTN_FAST_WEIGHTS
        return cls(out)

    def __getattr__(self, name):
        c = self.__dict__["_c"]
        if name in _ATTENTION_REQUIRED:
            return getattr(c, name)
        if hasattr(c.config.layout, name) and name != "reserved":
            return getattr(c.config.layout, name)
        if hasattr(c.config, name) and name != "reserved":
            return getattr(c.config, name)
        raise AttributeError(name)

    @property
    def layout(self):
        lay = self._c.config.layout
        return (lay.page_size, lay.page_stride_bytes, lay.key_in_page_offset,
                lay.value_in_page_offset, lay.key_row_bytes, lay.value_row_bytes)


def _paged_attention(fn, kernels, plan: PagedAttentionPlan, buffers: dict, max_sequence_length: int,
                     stream):
    b = _AttentionBuffers()
    for n in _ATTENTION_BUFFERS:
        buf = buffers[n]
        setattr(b, n, _DeviceBuffer(buf.ptr, buf.nbytes) if hasattr(buf, "nbytes") else buf)
        setattr(b, n + "_offset", buffers.get(n + "_offset", 0))
    _call(fn, kernels._h, ctypes.byref(plan._c), ctypes.byref(b), max_sequence_length,
          _stream(stream))


def synthetic_words(seed: int, word_index) -> np.ndarray:
    """Host copy of the words at `word_index` (8-byte word indices) of a
    FILL_BITS buffer: the splitmix64 stream the device fill writes."""
    i = np.asarray(word_index, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + (i + np.uint64(1)) * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


# --- bootstrap wire format (pd_bootstrap.rs) --------------------------------------------------

BOOTSTRAP_MAX_PARTS = 16
KV_POLL = {0: "Failed", 1: "Bootstrapping", 2: "WaitingForInput", 3: "Transferring", 4: "Success"}


def _ptr_list(ptr, n):
    return [ptr[i] for i in range(n)]


def _lists_out(l):
    return [[l.values[j] for j in range(l.offsets[i], l.offsets[i + 1])] for i in range(l.count)]


def _lists_in(lists, ctype, struct):
    """(struct, keep-alive arrays) for a list of lists."""
    values = [v for one in lists for v in one]
    offsets = [0]
    for one in lists:
        offsets.append(offsets[-1] + len(one))
    va = (ctype * max(1, len(values)))(*values)
    oa = (_u64 * len(offsets))(*offsets)
    return struct(ctypes.cast(va, ctypes.POINTER(ctype)), ctypes.cast(oa, ctypes.POINTER(_u64)), len(lists)), (va, oa)


class DecodeLayout:
    """A decode pool's geometry as the layout extension advertises it: a
    PagedKvCacheLayout, its head layout (NHD/HND) and head chunks per row."""

    def __init__(self, layout: "PagedKvCacheLayout", head_layout: int = NHD, heads: int = 0):
        self.layout, self.head_layout, self.heads = layout, head_layout, heads

    def _c(self) -> _DecodeLayout:
        return _DecodeLayout(self.layout._c, self.head_layout, 0, self.heads)

    @classmethod
    def _from_c(cls, p):
        if not p:
            return None
        d = p.contents
        c = _PagedLayout()
        ctypes.pointer(c)[0] = d.layout
        return cls(PagedKvCacheLayout(c), d.head_layout, d.heads)


def _frame_parts(frame):
    """(parts array, keep-alive buffers) for a list of bytes-like parts."""
    bufs = [ctypes.create_string_buffer(bytes(p), max(1, len(p))) for p in frame]
    parts = (_FramePart * max(1, len(frame)))(
        *[_FramePart(ctypes.cast(b, ctypes.c_void_p), len(p)) for b, p in zip(bufs, frame)])
    return parts, bufs


def _emit(fn, struct):
    needed, count = _u64(), ctypes.c_uint32()
    _call(fn, ctypes.byref(struct), None, 0, None, ctypes.byref(count), ctypes.byref(needed))
    buf = ctypes.create_string_buffer(max(1, needed.value))
    parts = (_FramePart * BOOTSTRAP_MAX_PARTS)()
    _call(fn, ctypes.byref(struct), ctypes.cast(buf, ctypes.c_void_p), needed.value, parts,
          ctypes.byref(count), ctypes.byref(needed))
    base = ctypes.addressof(buf)
    raw = buf.raw
    return [raw[parts[i].data - base: parts[i].data - base + parts[i].len] if parts[i].len else b""
            for i in range(count.value)]


def encode_kv_args_frame(*, endpoint: str, dst_port: int, mooncake_session_id: str, dst_kv_ptrs,
                         dst_aux_ptrs=(), dst_state_data_ptrs=(), dst_tp_rank: int = 0,
                         dst_attn_tp_size: int = 1, dst_kv_item_len: int = 0, dst_state_item_lens=(),
                         dst_state_dim_per_tensor=(), decode_layout: DecodeLayout | None = None):
    """MooncakeDecodeKvArgsRegistration::to_frame (pd_bootstrap.rs:685-706),
    plus the decode-layout part when `decode_layout` is given."""
    kp = (_u64 * max(1, len(dst_kv_ptrs)))(*dst_kv_ptrs)
    ap = (_u64 * max(1, len(dst_aux_ptrs)))(*dst_aux_ptrs)
    sd, k1 = _lists_in(dst_state_data_ptrs, _u64, _U64Lists)
    il, k2 = _lists_in(dst_state_item_lens, ctypes.c_uint32, _U32Lists)
    dp, k3 = _lists_in(dst_state_dim_per_tensor, ctypes.c_uint32, _U32Lists)
    dl = decode_layout._c() if decode_layout is not None else None
    a = _BootKvArgs(endpoint.encode(), mooncake_session_id.encode(), dst_port, dst_tp_rank, dst_attn_tp_size,
                    dst_kv_item_len, ctypes.cast(kp, ctypes.POINTER(_u64)), len(dst_kv_ptrs),
                    ctypes.cast(ap, ctypes.POINTER(_u64)), len(dst_aux_ptrs), sd, il, dp,
                    ctypes.pointer(dl) if dl is not None else None)
    return _emit(lib().sgl_kv_bootstrap_encode_kv_args, a)


def encode_transfer_frame(*, room: int, endpoint: str, dst_port: int, mooncake_session_id: str,
                          dst_kv_indices=(), dst_aux_index: int | None = 0, dst_state_indices=(),
                          required_dst_info_num: int = 1, decode_prefix_len: int | None = None,
                          is_dummy: bool = False):
    """MooncakeDecodeTransferMetadata::to_frame (pd_bootstrap.rs:720-749)."""
    ki = (ctypes.c_int32 * max(1, len(dst_kv_indices)))(*dst_kv_indices)
    si, keep = _lists_in(dst_state_indices, ctypes.c_int32, _I32Lists)
    t = _BootTransfer(room, endpoint.encode(), mooncake_session_id.encode(), dst_port, int(is_dummy),
                      ctypes.cast(ki, ctypes.POINTER(ctypes.c_int32)), len(dst_kv_indices),
                      0 if dst_aux_index is None else 1, dst_aux_index or 0, si, required_dst_info_num,
                      0 if decode_prefix_len is None else 1, 0, decode_prefix_len or 0)
    return _emit(lib().sgl_kv_bootstrap_encode_transfer, t)


class PrefillBootstrapState:
    """The Mooncake tables of PrefillBootstrapState (pd_bootstrap.rs:150-270)."""

    def __init__(self):
        h = ctypes.c_void_p()
        _call(lib().sgl_kv_bootstrap_create, ctypes.byref(h))
        self._h = h.value

    def close(self):
        if getattr(self, "_h", None):
            lib().sgl_kv_bootstrap_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def ingest_mooncake_bootstrap_frame(self, frame):
        parts, keep = _frame_parts(frame)
        _call(lib().sgl_kv_bootstrap_ingest, self._h, parts, len(frame))

    def decode_kv_args_registration_count(self) -> int:
        n = _u64()
        _call(lib().sgl_kv_bootstrap_registration_count, self._h, ctypes.byref(n))
        return n.value

    def decode_kv_args(self, session: str) -> dict:
        a = _BootKvArgs()
        _call(lib().sgl_kv_bootstrap_get_kv_args, self._h, session.encode(), ctypes.byref(a))
        return {"endpoint": a.endpoint.decode(), "dst_port": a.dst_port,
                "mooncake_session_id": a.mooncake_session_id.decode(),
                "dst_kv_ptrs": _ptr_list(a.dst_kv_ptrs, a.dst_kv_ptr_count),
                "dst_aux_ptrs": _ptr_list(a.dst_aux_ptrs, a.dst_aux_ptr_count),
                "dst_state_data_ptrs": _lists_out(a.dst_state_data_ptrs),
                "dst_tp_rank": a.dst_tp_rank, "dst_attn_tp_size": a.dst_attn_tp_size,
                "dst_kv_item_len": a.dst_kv_item_len,
                "dst_state_item_lens": _lists_out(a.dst_state_item_lens),
                "dst_state_dim_per_tensor": _lists_out(a.dst_state_dim_per_tensor),
                "decode_layout": DecodeLayout._from_c(a.decode_layout)}

    def transfer_status(self, room: int):
        st = ctypes.c_int32()
        _call(lib().sgl_kv_bootstrap_transfer_status, self._h, room, ctypes.byref(st))
        return None if st.value < 0 else KV_POLL[st.value]

    def transfer_room(self, room: int) -> dict:
        req, has, pre, n = _u64(), ctypes.c_uint32(), _u64(), _u64()
        _call(lib().sgl_kv_bootstrap_room, self._h, room, ctypes.byref(req), ctypes.byref(has),
              ctypes.byref(pre), ctypes.byref(n))
        return {"required_dst_info_num": req.value, "decode_prefix_len": pre.value if has.value else None,
                "transfer_count": n.value}

    def transfer(self, room: int, session: str) -> dict:
        t = _BootTransfer()
        _call(lib().sgl_kv_bootstrap_get_transfer, self._h, room, session.encode(), ctypes.byref(t))
        return {"room": t.room, "endpoint": t.endpoint.decode(), "dst_port": t.dst_port,
                "mooncake_session_id": t.mooncake_session_id.decode(), "is_dummy": bool(t.is_dummy),
                "dst_kv_indices": _ptr_list(t.dst_kv_indices, t.dst_kv_index_count),
                "dst_aux_index": t.dst_aux_index if t.has_dst_aux_index else None,
                "dst_state_indices": _lists_out(t.dst_state_indices),
                "required_dst_info_num": t.required_dst_info_num,
                "decode_prefix_len": t.decode_prefix_len if t.has_decode_prefix_len else None}

    def remote_kv_layouts_for_room(self, room: int):
        """[(session, {dst_kv_ptrs, dst_kv_indices, dst_kv_item_len, decode_layout})]."""
        n = _u64()
        _call(lib().sgl_kv_bootstrap_remote_layouts, self._h, room, None, 0, ctypes.byref(n))
        out = (_RemoteKvLayout * max(1, n.value))()
        _call(lib().sgl_kv_bootstrap_remote_layouts, self._h, room, out, n.value, ctypes.byref(n))
        return [(l.mooncake_session_id.decode(),
                 {"dst_kv_ptrs": _ptr_list(l.dst_kv_ptrs, l.dst_kv_ptr_count),
                  "dst_kv_indices": _ptr_list(l.dst_kv_indices, l.dst_kv_index_count),
                  "dst_kv_item_len": l.dst_kv_item_len,
                  "decode_layout": DecodeLayout._from_c(l.decode_layout)})
                for l in out[: n.value]]
