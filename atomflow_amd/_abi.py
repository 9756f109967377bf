"""ctypes prototypes of libatomflow_kv.so (include/af_kv.h, include/af_runtime.h)."""
import ctypes

P = ctypes.c_void_p
I = ctypes.c_int
I32 = ctypes.c_int32
I64 = ctypes.c_int64
U32 = ctypes.c_uint32
U64 = ctypes.c_uint64
F = ctypes.c_float
SZ = ctypes.c_size_t
PI32 = ctypes.POINTER(ctypes.c_int32)
PI64 = ctypes.POINTER(ctypes.c_int64)


class KvPool(ctypes.Structure):
    """af_kv_pool (include/af_kv.h)."""

    _fields_ = [
        ("base", P),
        ("scales", P),
        ("dtype", I32),
        ("block_size", I32),
        ("n_layers", I32),
        ("n_kv_heads", I32),
        ("head_dim", I32),
        ("flags", I32),
        ("total_blocks", I64),
    ]


PPOOL = ctypes.POINTER(KvPool)

PROTOTYPES = {
    # af_kv.h
    "af_status_string": (ctypes.c_char_p, [I]),
    "af_version": (I, []),
    "af_rope_table_build": (I, [P, P, I, I, F, P]),
    "af_rope_table_host": (I, [P, P, I, I, F]),
    "af_rope": (I, [P, P, P, P, I, I, I, I, P]),
    "af_write_kv_cache": (I, [P, P, P, I, I, I, I, P]),
    "af_rope_append": (I, [P, P, P, P, P, I, P, I, I, I, I, P, P]),
    "af_cached_attention": (I, [P, P, P, P, I, I, I, I, P]),
    "af_cached_attention_noalloc": (I, [P, P, P, P, I, I, I, I, P]),
    "af_cached_attention_noalloc_max_bytes": (SZ, []),
    "af_attention_reserve": (I, [I, I, I, I]),
    "af_attention_workspace_size": (SZ, [I, I, I, I, I]),
    "af_attention_workspace_init": (I, [P, SZ, P]),
    "af_attention_default_splits": (I, [I, I, I]),
    "af_cached_attention_ex": (I, [P, P, P, P, I, P, I, I, I, I, I, P, SZ, P]),
    "af_decode_attention_fused": (I, [P, P, P, P, P, I, P, I, P, I, I, I, I, P, SZ, P, P]),
    "af_paged_decode_fused": (I, [P, I, PPOOL, I, P, P, P, P, I, P, I, I, P, I, I, I, P, SZ, P]),
    "af_kv_pool_bytes": (SZ, [PPOOL]),
    "af_paged_rope_append": (I, [P, I, PPOOL, I, P, P, P, P, I, I, P]),
    "af_paged_attention": (I, [P, I, PPOOL, I, P, I, P, I, I, P, I, I, I, P, SZ, P]),
    "af_paged_attention_shared_prefix": (I, [P, I, PPOOL, I, P, I, I, P, I, P, I, I, P, I, I, I,
                                             P, SZ, P]),
    "af_paged_decode_fused_shared_prefix": (I, [P, I, PPOOL, I, P, P, P, P, I, P, I, I, P, I, I,
                                                P, I, I, I, P, SZ, P]),
    "af_paged_gather": (I, [PPOOL, I, P, I, P, P, P]),
    "af_kv_copy_blocks": (I, [PPOOL, P, P, I, P]),
    "af_fp8_quantize": (I, [P, P, SZ, F, P]),
    "af_w8a16_gemv": (I, [P, P, P, P, I, I, I, P]),
    "af_w8a16_gemm_batched": (I, [P, I64, I, P, P, P, I64, I, I, I, P]),
    "af_paged_qkv_rope_append": (I, [P, I64, I, P, P, I, I, P, P, I, P, P, P, P, I, I, P, P]),
    "af_w8a16_gemv_pair": (I, [P, P, P, P, I, P, P, P, I, I, I, P]),
    "af_qkv_rope_append": (I, [P, P, P, I, I, P, P, P, P, P, I, P, I, I, I, I, P, P]),
    "af_prefill_rope_append": (I, [P, I, P, P, P, P, I, P, I, I, I, I, P, P]),
    "af_prefill_attention": (I, [P, I, P, P, P, I, I, I, I, I, I, I, I, P]),
    "af_tiled_attention": (I, [P, P, P, P, I, I, I, I, I, P]),
    "af_paged_prefill_attention": (I, [P, I, P, I, P, I, I, I, I, P, I, I, P]),
    "af_prefill_attention_ws": (I, [P, I, P, P, P, I, I, I, I, I, I, I, I, I, P, SZ, P]),
    "af_paged_prefill_attention_ws": (I, [P, I, P, I, P, I, I, I, I, P, I, I, I, P, SZ, P]),
    "af_prefill_workspace_size": (SZ, [I, I, I, I, I]),
    "af_paged_prefill_attention_batched": (I, [P, I, P, I, P, I, P, P, I, P, I, I, P]),
    "af_prefill_tile_map": (I, [P, I, P, I]),
    "af_prefill_piece_map": (I, [P, I, I, I, P, I, P, P, P]),
    "af_paged_prefill_attention_batched_ws": (I, [P, I, P, I, P, I, P, P, I, I, I, P, I, I, P, SZ, P]),
    "af_weights_open": (I, [ctypes.c_char_p, P]),
    "af_weights_close": (I, [P]),
    "af_weights_layout_bytes": (SZ, [P]),
    "af_weights_header": (I, [P, P]),
    "af_weights_payload_bytes": (SZ, [P]),
    "af_weights_tensor": (I, [P, I, I, P, P, P]),
    "af_weights_upload": (I, [P, P, SZ, P]),
    "af_sched_create": (I, [P, I, I, I, I, P]),
    "af_sched_destroy": (I, [P]),
    "af_sched_add_request": (I, [P, I64, I, I]),
    "af_sched_add_request_prefix": (I, [P, I64, I, I, I64, I]),
    "af_sched_set_prefix_cache": (I, [P, I]),
    "af_sched_clear_prefix_cache": (I, [P]),
    "af_sched_plan_prefix": (I, [P, P, P, P, P]),
    "af_sched_step": (I, [P, P]),
    "af_sched_plan_decode": (I, [P, P, P, P, P]),
    "af_sched_plan_decode_shared": (I, [P, P, P]),
    "af_sched_plan_prefill": (I, [P, P, P, P, P]),
    "af_sched_plan_copies": (I, [P, P]),
    "af_sched_plan_events": (I, [P, P, P]),
    "af_bm_create": (I, [I, I, I, I, I, I, I, ctypes.POINTER(P)]),
    "af_bm_destroy": (I, [P]),
    "af_bm_attach_pool": (I, [P, P, P]),
    "af_bm_pool": (I, [P, PPOOL]),
    "af_bm_allocate_block": (I, [P]),
    "af_bm_free_block": (I, [P, I]),
    "af_bm_num_free_blocks": (I, [P]),
    "af_bm_ref_count": (I, [P, I]),
    "af_bm_hold_copy_source": (I, [P, I]),
    "af_bm_release_copy_sources": (I, [P]),
    "af_bm_seq_create": (I, [P]),
    "af_bm_seq_fork": (I, [P, I]),
    "af_bm_seq_free": (I, [P, I]),
    "af_bm_seq_len": (I, [P, I]),
    "af_bm_seq_table": (I, [P, I, PI32, I, PI32]),
    "af_bm_seq_append": (I, [P, I, PI64, PI32, PI32, PI32]),
    "af_bm_seq_extend": (I, [P, I, I, PI32, PI32, PI32]),
    "af_bm_seq_slot": (I64, [P, I, I]),
    "af_bm_plan_decode": (I, [P, P, I, P, P, P, I, PI32]),
    "af_bm_export_tables": (I, [P, P, I, P, I, P]),
    # af_runtime.h
    "af_rt_device_count": (I, [ctypes.POINTER(I)]),
    "af_rt_set_device": (I, [I]),
    "af_rt_device_info": (I, [ctypes.c_char_p, I, ctypes.POINTER(I), ctypes.c_char_p, I]),
    "af_rt_device_sync": (I, []),
    "af_rt_last_error": (I, []),
    "af_rt_malloc": (I, [ctypes.POINTER(P), SZ]),
    "af_rt_free": (I, [P]),
    "af_rt_host_malloc": (I, [ctypes.POINTER(P), SZ]),
    "af_rt_host_free": (I, [P]),
    "af_rt_mem_info": (I, [ctypes.POINTER(SZ), ctypes.POINTER(SZ)]),
    "af_rt_memcpy_h2d": (I, [P, P, SZ, P]),
    "af_rt_memcpy_d2h": (I, [P, P, SZ, P]),
    "af_rt_memcpy_d2d": (I, [P, P, SZ, P]),
    "af_rt_fill_u32": (I, [P, U32, SZ, P]),
    "af_rt_add_i32": (I, [P, I, I32, P]),
    "af_rt_read_probe": (I, [P, SZ, I, I, I, I, P, P]),
    "af_rt_fill_randn_f16": (I, [P, SZ, U64, F, P]),
    "af_rt_fill_randn_fp8": (I, [P, SZ, U64, F, P]),
    "af_rt_stream_create": (I, [ctypes.POINTER(P)]),
    "af_rt_stream_destroy": (I, [P]),
    "af_rt_stream_sync": (I, [P]),
    "af_rt_event_create": (I, [ctypes.POINTER(P)]),
    "af_rt_event_destroy": (I, [P]),
    "af_rt_event_record": (I, [P, P]),
    "af_rt_event_sync": (I, [P]),
    "af_rt_event_elapsed_ms": (I, [ctypes.POINTER(F), P, P]),
    "af_rt_capture_begin": (I, [P]),
    "af_rt_capture_end": (I, [P, ctypes.POINTER(P)]),
    "af_rt_graph_launch": (I, [P, P]),
    "af_rt_graph_destroy": (I, [P]),
}


def bind(lib):
    for name, (res, args) in PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib
