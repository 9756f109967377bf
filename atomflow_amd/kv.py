"""Python mirror of the KV-cache operator interface.

Names, argument order and meaning follow the reference's launchers
(include/ops/kernel.h:32-42, 93-103, 167-174, 195-197) and its paged contract
(src/experimental/server_arch/paged_kv_manager.h:90-121). Tensors are device
pointers (``int``) or ``device.DeviceBuffer`` objects; ``stream`` is a
``device.Stream``, a raw handle, or None (default stream). Every call goes to
libatomflow_kv.so and raises ``AfError`` on a non-zero status.
"""
import ctypes

import numpy as np

from . import AF_KV_FP16, AF_KV_FP8_E4M3, AfError, _abi, check, lib
from .device import DeviceBuffer, _s


def _p(x):
    if x is None:
        return None
    return x.ptr if isinstance(x, DeviceBuffer) else int(x)


# ---- a1 / a2 / a3 ---------------------------------------------------------
def build_rope_cache(d_cos, d_sin, max_seq, head_dim, base, stream=None):
    check(lib().af_rope_table_build(_p(d_cos), _p(d_sin), max_seq, head_dim, base, _s(stream)),
          "build_rope_cache")


def rope_table_host(max_seq, head_dim, base=500000.0):
    cos = np.empty((max_seq, head_dim // 2), np.float32)
    sin = np.empty((max_seq, head_dim // 2), np.float32)
    check(lib().af_rope_table_host(cos.ctypes.data, sin.ctypes.data, max_seq, head_dim, base),
          "af_rope_table_host")
    return cos, sin


def launch_rope(q, k, cos_cache, sin_cache, seq_len, kv_head_num, q_head_num, head_dim,
                stream=None):
    check(lib().af_rope(_p(q), _p(k), _p(cos_cache), _p(sin_cache), seq_len, kv_head_num,
                        q_head_num, head_dim, _s(stream)), "launch_rope")


def launch_write_kv_cache(qkv_out, k_cache, v_cache, current_pos, q_dim, kv_dim, max_seq,
                          stream=None):
    check(lib().af_write_kv_cache(_p(qkv_out), _p(k_cache), _p(v_cache), current_pos, max_seq,
                                  q_dim, kv_dim, _s(stream)), "launch_write_kv_cache")


def launch_rope_append(qkv_out, k_cache, v_cache, cos_table, sin_table, pos, max_seq, n_q_heads,
                       n_kv_heads, head_dim, d_pos=None, d_status=None, stream=None):
    check(lib().af_rope_append(_p(qkv_out), _p(k_cache), _p(v_cache), _p(cos_table),
                               _p(sin_table), pos, _p(d_pos), max_seq, n_q_heads, n_kv_heads,
                               head_dim, _p(d_status), _s(stream)), "launch_rope_append")


# ---- W8A16 GEMV (qkv_gemm.cu launch_w8a16_gemv) and the fused QKV step -------
def launch_w8a16_gemv(x, weight, scales, y, n, k, group_size=128, stream=None):
    """y[n] = sum_k e4m3(weight[n,k]) * scales[n, k/group_size] * x[k] (fp16 out)."""
    check(lib().af_w8a16_gemv(_p(x), _p(weight), _p(scales), _p(y), n, k, group_size, _s(stream)),
          "launch_w8a16_gemv")


def launch_w8a16_gemv_pair(x, w0, s0, y0, n0, w1, s1, y1, n1, k, group_size=128, stream=None):
    """y0 = W0 x and y1 = W1 x in one launch (gate and up), each as launch_w8a16_gemv."""
    check(lib().af_w8a16_gemv_pair(_p(x), _p(w0), _p(s0), _p(y0), n0, _p(w1), _p(s1), _p(y1), n1,
                                   k, group_size, _s(stream)), "launch_w8a16_gemv_pair")


def launch_w8a16_gemm_batched(x, x_stride, m, weight, scales, y, y_stride, n, k, group_size=128,
                              stream=None):
    """y[i] = W x[i] for m tokens (rows x_stride / y_stride elements apart), one launch."""
    check(lib().af_w8a16_gemm_batched(_p(x), x_stride, m, _p(weight), _p(scales), _p(y), y_stride,
                                      n, k, group_size, _s(stream)), "launch_w8a16_gemm_batched")


def launch_paged_qkv_rope_append(x, x_stride, m, w_qkv, scales, k, qkv_out, pool, layer, d_slots,
                                 d_positions, cos_table, sin_table, max_pos, n_q_heads,
                                 group_size=128, d_status=None, stream=None):
    """Batched QKV projection + RoPE + paged append (af_paged_qkv_rope_append)."""
    check(lib().af_paged_qkv_rope_append(_p(x), x_stride, m, _p(w_qkv), _p(scales), k, group_size,
                                         _p(qkv_out), ctypes.byref(pool), layer, _p(d_slots),
                                         _p(d_positions), _p(cos_table), _p(sin_table), max_pos,
                                         n_q_heads, _p(d_status), _s(stream)),
          "launch_paged_qkv_rope_append")


def launch_qkv_rope_append(x, w_qkv, scales, k, qkv_out, k_cache, v_cache, cos_table, sin_table,
                           pos, max_seq, n_q_heads, n_kv_heads, head_dim, group_size=128,
                           d_pos=None, d_status=None, stream=None):
    """QKV projection into qkv_out, RoPE of Q and K, K/V appended at row pos."""
    check(lib().af_qkv_rope_append(_p(x), _p(w_qkv), _p(scales), k, group_size, _p(qkv_out),
                                   _p(k_cache), _p(v_cache), _p(cos_table), _p(sin_table), pos,
                                   _p(d_pos), max_seq, n_q_heads, n_kv_heads, head_dim,
                                   _p(d_status), _s(stream)), "launch_qkv_rope_append")


# ---- prefill (multi-token append, causal attention over a prompt chunk) -----
def launch_prefill_rope_append(qkv_out, n, k_cache, v_cache, cos_table, sin_table, p0, max_seq,
                               n_q_heads, n_kv_heads, head_dim, d_p0=None, d_status=None,
                               stream=None):
    """RoPE of n qkv rows at positions p0.. and their K/V written to cache rows p0.."""
    check(lib().af_prefill_rope_append(_p(qkv_out), n, _p(k_cache), _p(v_cache), _p(cos_table),
                                       _p(sin_table), p0, _p(d_p0), max_seq, n_q_heads,
                                       n_kv_heads, head_dim, _p(d_status), _s(stream)),
          "launch_prefill_rope_append")


def launch_prefill_attention(q, q_stride, k_cache, v_cache, out, out_stride, p0, n, kv_len,
                             max_seq, n_q_heads, n_kv_heads, head_dim, stream=None):
    """Causal attention: query i attends cache rows [0, min(p0 + i + 1, kv_len))."""
    check(lib().af_prefill_attention(_p(q), q_stride, _p(k_cache), _p(v_cache), _p(out),
                                     out_stride, p0, n, kv_len, max_seq, n_q_heads, n_kv_heads,
                                     head_dim, _s(stream)), "launch_prefill_attention")


def launch_paged_prefill_attention(q, q_stride, pool, layer, d_block_table, max_blocks, p0, n,
                                   kv_len, out, out_stride, n_q_heads, stream=None):
    """Causal chunk attention over one sequence's rows of a paged pool."""
    check(lib().af_paged_prefill_attention(_p(q), q_stride, ctypes.byref(pool), layer,
                                           _p(d_block_table), max_blocks, p0, n, kv_len, _p(out),
                                           out_stride, n_q_heads, _s(stream)),
          "launch_paged_prefill_attention")


def _ws(workspace):
    """(pointer, bytes) of a workspace object, or (None, 0)."""
    return (None, 0) if workspace is None else (workspace.ptr, workspace.nbytes)


class PrefillWorkspace:
    """Key-piece workspace of one chunk shape (records + arrival counters),
    zeroed once at creation; launches that share it must be ordered."""

    def __init__(self, p0, n, kv_len, n_q_heads, key_pieces=0, stream=None):
        self.nbytes = lib().af_prefill_workspace_size(p0, n, kv_len, n_q_heads, key_pieces)
        if self.nbytes == 0:
            raise AfError(-2, "af_prefill_workspace_size")
        self.buf = DeviceBuffer(self.nbytes)
        check(lib().af_attention_workspace_init(self.buf.ptr, self.nbytes, _s(stream)),
              "af_attention_workspace_init")

    @property
    def ptr(self):
        return self.buf.ptr


def launch_prefill_attention_ws(q, q_stride, k_cache, v_cache, out, out_stride, p0, n, kv_len,
                                max_seq, n_q_heads, n_kv_heads, head_dim, workspace, key_pieces=0,
                                stream=None):
    """launch_prefill_attention with heavy query tiles cut into key pieces."""
    check(lib().af_prefill_attention_ws(_p(q), q_stride, _p(k_cache), _p(v_cache), _p(out),
                                        out_stride, p0, n, kv_len, max_seq, n_q_heads, n_kv_heads,
                                        head_dim, key_pieces, *_ws(workspace), _s(stream)),
          "launch_prefill_attention_ws")


def launch_paged_prefill_attention_ws(q, q_stride, pool, layer, d_block_table, max_blocks, p0, n,
                                      kv_len, out, out_stride, n_q_heads, workspace, key_pieces=0,
                                      stream=None):
    """launch_paged_prefill_attention with heavy query tiles cut into key pieces."""
    check(lib().af_paged_prefill_attention_ws(_p(q), q_stride, ctypes.byref(pool), layer,
                                              _p(d_block_table), max_blocks, p0, n, kv_len, _p(out),
                                              out_stride, n_q_heads, key_pieces, *_ws(workspace),
                                              _s(stream)), "launch_paged_prefill_attention_ws")


def prefill_tile_map(chunks):
    """(chunk, tile) pairs of the chunks [(p0, n, kv_len, row0), ...], heaviest first."""
    ch = np.ascontiguousarray(chunks, np.int32).reshape(-1, 4)
    max_tiles = int(sum((int(n) + 127) // 128 for n in ch[:, 1])) + 1
    out = np.zeros((max_tiles, 2), np.int32)
    n = lib().af_prefill_tile_map(ch.ctypes.data, len(ch), out.ctypes.data, max_tiles)
    if n < 0:
        raise AfError(n, "af_prefill_tile_map")
    return out[:n].copy()


def launch_paged_prefill_attention_batched(q, q_stride, pool, layer, d_tables, max_blocks,
                                           d_chunks, d_tile_map, n_tiles, out, out_stride,
                                           n_q_heads, stream=None):
    """Chunked prefill of several sequences in one launch (see af_kv.h)."""
    check(lib().af_paged_prefill_attention_batched(
        _p(q), q_stride, ctypes.byref(pool), layer, _p(d_tables), max_blocks, _p(d_chunks),
        _p(d_tile_map), n_tiles, _p(out), out_stride, n_q_heads, _s(stream)),
        "launch_paged_prefill_attention_batched")


def prefill_piece_map(chunks, n_q_heads, key_pieces=0):
    """Key-piece map of the chunks [(p0, n, kv_len, row0), ...]: (entries [n][4],
    n_groups, max_pieces, workspace bytes), heaviest piece first."""
    ch = np.ascontiguousarray(chunks, np.int32).reshape(-1, 4)
    max_entries = 4 * int(sum((int(n) + 127) // 128 for n in ch[:, 1])) + 1
    out = np.zeros((max_entries, 4), np.int32)
    groups, most, nbytes = ctypes.c_int(), ctypes.c_int(), ctypes.c_size_t()
    n = lib().af_prefill_piece_map(ch.ctypes.data, len(ch), n_q_heads, key_pieces,
                                   out.ctypes.data, max_entries, ctypes.byref(groups),
                                   ctypes.byref(most), ctypes.byref(nbytes))
    if n < 0:
        raise AfError(n, "af_prefill_piece_map")
    return out[:n].copy(), groups.value, most.value, nbytes.value


class RecordWorkspace:
    """A key-piece workspace of a given size, zeroed once at creation."""

    def __init__(self, nbytes, stream=None):
        self.nbytes = max(int(nbytes), 64 * 1024)
        self.buf = DeviceBuffer(self.nbytes)
        check(lib().af_attention_workspace_init(self.buf.ptr, self.nbytes, _s(stream)),
              "af_attention_workspace_init")

    @property
    def ptr(self):
        return self.buf.ptr


def launch_paged_prefill_attention_batched_ws(q, q_stride, pool, layer, d_tables, max_blocks,
                                              d_chunks, d_piece_map, n_entries, n_groups,
                                              max_pieces, out, out_stride, n_q_heads, workspace,
                                              stream=None):
    """launch_paged_prefill_attention_batched over a key-piece map."""
    check(lib().af_paged_prefill_attention_batched_ws(
        _p(q), q_stride, ctypes.byref(pool), layer, _p(d_tables), max_blocks, _p(d_chunks),
        _p(d_piece_map), n_entries, n_groups, max_pieces, _p(out), out_stride, n_q_heads,
        *_ws(workspace), _s(stream)), "launch_paged_prefill_attention_batched_ws")


def launch_tiled_attention_kernel(q, k, v, out, seq_q, seq_kv, head_dim, n_q_heads, n_kv_heads,
                                  stream=None):
    """tiled_attention.cu launch_tiled_attention_kernel<half>: query i attends keys s <= i."""
    check(lib().af_tiled_attention(_p(q), _p(k), _p(v), _p(out), seq_q, seq_kv, head_dim,
                                   n_q_heads, n_kv_heads, _s(stream)),
          "launch_tiled_attention_kernel")


# ---- a5 ---------------------------------------------------------------------
def launch_cached_attention(q, k_cache, v_cache, out, seq_len, head_dim, n_q_heads, n_kv_heads,
                            stream=None):
    check(lib().af_cached_attention(_p(q), _p(k_cache), _p(v_cache), _p(out), seq_len, head_dim,
                                    n_q_heads, n_kv_heads, _s(stream)), "launch_cached_attention")


def default_splits(max_seq_len, batch, n_kv_heads):
    return lib().af_attention_default_splits(max_seq_len, batch, n_kv_heads)


class AttentionWorkspace:
    """Split-K workspace (partials + arrival counters), zeroed once at creation."""

    def __init__(self, batch, n_q_heads, n_kv_heads, head_dim, num_splits=0, stream=None):
        self.nbytes = lib().af_attention_workspace_size(batch, n_q_heads, n_kv_heads, head_dim,
                                                        num_splits)
        if self.nbytes == 0:
            raise AfError(-2, "af_attention_workspace_size")
        self.buf = DeviceBuffer(self.nbytes)
        self.reset(stream)

    def reset(self, stream=None):
        """Zero the counters again (clears the poison a timed-out combiner leaves)."""
        check(lib().af_attention_workspace_init(self.buf.ptr, self.nbytes, _s(stream)),
              "af_attention_workspace_init")

    @property
    def ptr(self):
        return self.buf.ptr


def launch_cached_attention_ex(q, k_cache, v_cache, out, seq_len, max_seq_len, head_dim,
                               n_q_heads, n_kv_heads, workspace, num_splits=0, d_seq_len=None,
                               stream=None):
    check(lib().af_cached_attention_ex(_p(q), _p(k_cache), _p(v_cache), _p(out), seq_len,
                                       _p(d_seq_len), max_seq_len, head_dim, n_q_heads,
                                       n_kv_heads, num_splits, workspace.ptr, workspace.nbytes,
                                       _s(stream)), "launch_cached_attention_ex")


def launch_decode_attention_fused(qkv_out, k_cache, v_cache, cos_table, sin_table, pos, max_seq,
                                  out, n_q_heads, n_kv_heads, head_dim, workspace, num_splits=0,
                                  d_pos=None, d_status=None, stream=None):
    """launch_rope_append(pos) + attention over pos + 1 tokens, one kernel."""
    check(lib().af_decode_attention_fused(_p(qkv_out), _p(k_cache), _p(v_cache), _p(cos_table),
                                          _p(sin_table), pos, _p(d_pos), max_seq, _p(out),
                                          n_q_heads, n_kv_heads, head_dim, num_splits,
                                          workspace.ptr, workspace.nbytes, _p(d_status),
                                          _s(stream)), "launch_decode_attention_fused")


# ---- a6-a8: paged pool -----------------------------------------------------
def make_pool(base, dtype, block_size, n_layers, n_kv_heads, head_dim, total_blocks, scales=None,
              flags=0):
    """af_kv_pool over `base`. flags: AF_KV_POOL_SHARED_BLOCKS when the block tables of one
    launch may map a block for several sequences (forks, prefix caching)."""
    p = _abi.KvPool()
    p.base = _p(base)
    p.scales = _p(scales)
    p.dtype = dtype
    p.block_size = block_size
    p.n_layers = n_layers
    p.n_kv_heads = n_kv_heads
    p.head_dim = head_dim
    p.flags = flags
    p.total_blocks = total_blocks
    return p


def pool_bytes(pool):
    return lib().af_kv_pool_bytes(ctypes.byref(pool))


def launch_paged_rope_append(qkv_out, batch, pool, layer, d_slots, d_positions, cos_table,
                             sin_table, max_pos, n_q_heads, stream=None):
    check(lib().af_paged_rope_append(_p(qkv_out), batch, ctypes.byref(pool), layer, _p(d_slots),
                                     _p(d_positions), _p(cos_table), _p(sin_table), max_pos,
                                     n_q_heads, _s(stream)), "launch_paged_rope_append")


def launch_paged_attention(q, q_stride, pool, layer, d_block_tables, max_blocks_per_seq,
                           d_seq_lens, batch, max_seq_len, out, out_stride, n_q_heads, workspace,
                           num_splits=0, stream=None):
    check(lib().af_paged_attention(_p(q), q_stride, ctypes.byref(pool), layer, _p(d_block_tables),
                                   max_blocks_per_seq, _p(d_seq_lens), batch, max_seq_len, _p(out),
                                   out_stride, n_q_heads, num_splits, workspace.ptr,
                                   workspace.nbytes, _s(stream)), "launch_paged_attention")


def launch_paged_decode_fused(qkv_out, batch, pool, layer, d_slots, d_positions, cos_table,
                              sin_table, max_pos, d_block_tables, max_blocks_per_seq, max_seq_len,
                              out, out_stride, n_q_heads, workspace, num_splits=0, stream=None):
    """Paged RoPE+append then attention (lengths = positions + 1), one kernel."""
    check(lib().af_paged_decode_fused(_p(qkv_out), batch, ctypes.byref(pool), layer, _p(d_slots),
                                      _p(d_positions), _p(cos_table), _p(sin_table), max_pos,
                                      _p(d_block_tables), max_blocks_per_seq, max_seq_len, _p(out),
                                      out_stride, n_q_heads, num_splits, workspace.ptr,
                                      workspace.nbytes, _s(stream)), "launch_paged_decode_fused")


def launch_paged_attention_shared_prefix(q, q_stride, pool, layer, d_prefix_table, prefix_len,
                                         d_block_tables, max_blocks_per_seq, d_seq_lens, batch,
                                         max_seq_len, out, out_stride, n_q_heads, workspace,
                                         num_splits=0, prefix_splits=0, stream=None):
    """af_paged_attention for sequences sharing rows [0, prefix_len): the prefix is
    attended once for the batch on the matrix cores, the rest per sequence."""
    check(lib().af_paged_attention_shared_prefix(
        _p(q), q_stride, ctypes.byref(pool), layer, _p(d_prefix_table), prefix_len, prefix_splits,
        _p(d_block_tables), max_blocks_per_seq, _p(d_seq_lens), batch, max_seq_len, _p(out),
        out_stride, n_q_heads, num_splits, workspace.ptr, workspace.nbytes, _s(stream)),
        "launch_paged_attention_shared_prefix")


def launch_paged_decode_fused_shared_prefix(qkv_out, batch, pool, layer, d_slots, d_positions,
                                            cos_table, sin_table, max_pos, d_prefix_table,
                                            prefix_len, d_block_tables, max_blocks_per_seq,
                                            max_seq_len, out, out_stride, n_q_heads, workspace,
                                            num_splits=0, prefix_splits=0, stream=None):
    """launch_paged_decode_fused with a shared prefix (two launches)."""
    check(lib().af_paged_decode_fused_shared_prefix(
        _p(qkv_out), batch, ctypes.byref(pool), layer, _p(d_slots), _p(d_positions),
        _p(cos_table), _p(sin_table), max_pos, _p(d_prefix_table), prefix_len, prefix_splits,
        _p(d_block_tables), max_blocks_per_seq, max_seq_len, _p(out), out_stride, n_q_heads,
        num_splits, workspace.ptr, workspace.nbytes, _s(stream)),
        "launch_paged_decode_fused_shared_prefix")


def paged_gather(pool, layer, d_block_table, seq_len, k_dst, v_dst, stream=None):
    check(lib().af_paged_gather(ctypes.byref(pool), layer, _p(d_block_table), seq_len, _p(k_dst),
                                _p(v_dst), _s(stream)), "paged_gather")


def kv_copy_blocks(pool, d_copies, d_count, max_copies, stream=None):
    check(lib().af_kv_copy_blocks(ctypes.byref(pool), _p(d_copies), _p(d_count), max_copies,
                                  _s(stream)), "kv_copy_blocks")


def fp8_quantize(src_f16, dst, n, scale, stream=None):
    check(lib().af_fp8_quantize(_p(src_f16), _p(dst), n, scale, _s(stream)), "fp8_quantize")


class BlockManager:
    """atomflow::server::BlockManager through the C ABI.

    ``allocate_block`` returns an id or -1 (pool exhausted) like the reference
    (paged_kv_manager.h:105-107); the other methods raise ``AfError``.
    """

    def __init__(self, total_blocks, block_size=16, n_layers=1, n_kv_heads=8, head_dim=128,
                 dtype=AF_KV_FP16, allocate_pool=False):
        h = ctypes.c_void_p()
        check(lib().af_bm_create(total_blocks, block_size, n_layers, n_kv_heads, head_dim, dtype,
                                 1 if allocate_pool else 0, ctypes.byref(h)), "af_bm_create")
        self.h = h.value
        self.block_size = block_size

    def close(self):
        """Destroys the manager, after every Scheduler built on it (a scheduler's
        teardown frees its cached sequences through the manager)."""
        for sched in list(getattr(self, "_schedulers", ())):
            sched.close()
        if self.h:
            lib().af_bm_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # reference contract
    def allocate_block(self):
        return lib().af_bm_allocate_block(self.h)

    def free_block(self, block_id):
        return check(lib().af_bm_free_block(self.h, block_id), "free_block")

    def num_free_blocks(self):
        return lib().af_bm_num_free_blocks(self.h)

    # extensions
    def try_free_block(self, block_id):
        return lib().af_bm_free_block(self.h, block_id)

    def ref_count(self, block_id):
        return lib().af_bm_ref_count(self.h, block_id)

    def hold_copy_source(self, block_id):
        return lib().af_bm_hold_copy_source(self.h, block_id)

    def release_copy_sources(self):
        return check(lib().af_bm_release_copy_sources(self.h), "release_copy_sources")

    def attach_pool(self, base, scales=None):
        check(lib().af_bm_attach_pool(self.h, _p(base), _p(scales)), "attach_pool")

    def pool(self):
        p = _abi.KvPool()
        check(lib().af_bm_pool(self.h, ctypes.byref(p)), "af_bm_pool")
        return p

    def seq_create(self):
        return _nonneg(lib().af_bm_seq_create(self.h), "seq_create")

    def seq_fork(self, src):
        return lib().af_bm_seq_fork(self.h, src)

    def seq_free(self, seq):
        return lib().af_bm_seq_free(self.h, seq)

    def seq_len(self, seq):
        return lib().af_bm_seq_len(self.h, seq)

    def seq_table(self, seq):
        n = lib().af_bm_seq_table(self.h, seq, None, 0, None)
        if n < 0:
            return n
        ids = (ctypes.c_int32 * max(n, 1))()
        fill = ctypes.c_int32(0)
        lib().af_bm_seq_table(self.h, seq, ids, n, ctypes.byref(fill))
        return list(ids[:n]), fill.value

    def seq_append(self, seq):
        """(pos, slot, (cow_src, cow_dst, cow_rows)) or a negative status."""
        slot = ctypes.c_int64(0)
        a, b, c = ctypes.c_int32(0), ctypes.c_int32(0), ctypes.c_int32(0)
        r = lib().af_bm_seq_append(self.h, seq, ctypes.byref(slot), ctypes.byref(a),
                                   ctypes.byref(b), ctypes.byref(c))
        if r < 0:
            return r
        return r, slot.value, (a.value, b.value, c.value)

    def seq_extend(self, seq, n):
        a, b, c = ctypes.c_int32(0), ctypes.c_int32(0), ctypes.c_int32(0)
        r = lib().af_bm_seq_extend(self.h, seq, n, ctypes.byref(a), ctypes.byref(b),
                                   ctypes.byref(c))
        if r < 0:
            return r
        return r, (a.value, b.value, c.value)

    def seq_slot(self, seq, pos):
        return lib().af_bm_seq_slot(self.h, seq, pos)

    def plan_decode(self, seqs, max_copies=None):
        """(slots[int64], positions[int32], copies[n,3] int32) or a negative status."""
        seqs = np.ascontiguousarray(seqs, np.int32)
        n = len(seqs)
        if max_copies is None:
            max_copies = max(n, 1)
        slots = np.zeros(n, np.int64)
        pos = np.zeros(n, np.int32)
        copies = np.zeros((max_copies, 3), np.int32)
        nc = ctypes.c_int32(0)
        r = lib().af_bm_plan_decode(self.h, seqs.ctypes.data, n, slots.ctypes.data, pos.ctypes.data,
                                    copies.ctypes.data, max_copies, ctypes.byref(nc))
        if r < 0:
            return r
        return slots, pos, copies[: nc.value].copy()

    def export_tables(self, seqs, max_blocks):
        seqs = np.ascontiguousarray(seqs, np.int32)
        tables = np.zeros((len(seqs), max_blocks), np.int32)
        lens = np.zeros(len(seqs), np.int32)
        check(lib().af_bm_export_tables(self.h, seqs.ctypes.data, len(seqs), tables.ctypes.data,
                                        max_blocks, lens.ctypes.data), "export_tables")
        return tables, lens


class Scheduler:
    """Continuous-batching scheduler (af_sched_*) over a BlockManager.

    ``step()`` returns the plan as a dict: finished / preempted request ids,
    decode [(request, seq, slot, position)], copies [(src, dst, rows)], prefill
    [(request, seq, p0, n, last, slots)], and the running / waiting counts;
    ``arrays`` also holds each decode entry's share group (-1: none) and shared
    rows (af_sched_plan_decode_shared).
    """

    def __init__(self, bm, max_running, max_step_tokens, prefill_chunk, watermark=0,
                 max_cached_prefixes=0):
        h = ctypes.c_void_p()
        check(lib().af_sched_create(bm.h, max_running, max_step_tokens, prefill_chunk, watermark,
                                    ctypes.byref(h)), "af_sched_create")
        self.h = h.value
        self.bm = bm  # keeps the manager alive
        # Strong references both ways: whichever finaliser runs first (the garbage
        # collector picks the order within a cycle) tears the scheduler down first.
        if not hasattr(bm, "_schedulers"):
            bm._schedulers = []
        bm._schedulers.append(self)
        if max_cached_prefixes:
            self.set_prefix_cache(max_cached_prefixes)

    def set_prefix_cache(self, max_entries):
        check(lib().af_sched_set_prefix_cache(self.h, max_entries), "af_sched_set_prefix_cache")

    def clear_prefix_cache(self):
        check(lib().af_sched_clear_prefix_cache(self.h), "af_sched_clear_prefix_cache")

    def close(self):
        if self.h:
            lib().af_sched_destroy(self.h)
            self.h = None
        owners = getattr(self.bm, "_schedulers", [])
        if self in owners:
            owners.remove(self)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def add_request(self, rid, prompt_len, max_new_tokens, prefix_key=-1, prefix_len=0):
        if prefix_len:
            return lib().af_sched_add_request_prefix(self.h, rid, prompt_len, max_new_tokens,
                                                     prefix_key, prefix_len) == 0
        return lib().af_sched_add_request(self.h, rid, prompt_len, max_new_tokens) == 0

    def step(self):
        c = np.zeros(8, np.int32)
        check(lib().af_sched_step(self.h, c.ctypes.data), "af_sched_step")
        nd, nc, nt, ncp, nf, npre, nrun, nwait = (int(x) for x in c)
        dreq, dseq = np.zeros(nd, np.int64), np.zeros(nd, np.int32)
        dslot, dpos = np.zeros(nd, np.int64), np.zeros(nd, np.int32)
        lib().af_sched_plan_decode(self.h, dreq.ctypes.data, dseq.ctypes.data, dslot.ctypes.data,
                                   dpos.ctypes.data)
        dgrp, drows = np.zeros(nd, np.int64), np.zeros(nd, np.int32)
        lib().af_sched_plan_decode_shared(self.h, dgrp.ctypes.data, drows.ctypes.data)
        preq, chunks = np.zeros(nc, np.int64), np.zeros((nc, 5), np.int32)
        pslot, ppos = np.zeros(nt, np.int64), np.zeros(nt, np.int32)
        lib().af_sched_plan_prefill(self.h, preq.ctypes.data, chunks.ctypes.data,
                                    pslot.ctypes.data, ppos.ctypes.data)
        copies = np.zeros((ncp, 3), np.int32)
        lib().af_sched_plan_copies(self.h, copies.ctypes.data)
        fin, pre = np.zeros(nf, np.int64), np.zeros(npre, np.int64)
        lib().af_sched_plan_events(self.h, fin.ctypes.data, pre.ctypes.data)
        prefill = []
        for i in range(nc):
            seq, p0, n, off, last = (int(x) for x in chunks[i])
            prefill.append((int(preq[i]), seq, p0, n, bool(last), [int(x) for x in pslot[off:off + n]]))
        pc = np.zeros(4, np.int32)
        lib().af_sched_plan_prefix(self.h, pc.ctypes.data, None, None, None)
        hits, cached, evicted = (np.zeros(int(x), np.int64) for x in pc[:3])
        lib().af_sched_plan_prefix(self.h, None, hits.ctypes.data, cached.ctypes.data,
                                   evicted.ctypes.data)
        return {
            "finished": [int(x) for x in fin], "preempted": [int(x) for x in pre],
            "decode": [(int(dreq[i]), int(dseq[i]), int(dslot[i]), int(dpos[i])) for i in range(nd)],
            "decode_shared": [(int(dgrp[i]), int(drows[i])) for i in range(nd)],
            "copies": [tuple(int(x) for x in row) for row in copies],
            "prefill": prefill, "running": nrun, "waiting": nwait,
            "prefix_hits": [int(x) for x in hits], "cached": [int(x) for x in cached],
            "evicted": [int(x) for x in evicted], "cache_entries": int(pc[3]),
            "arrays": {"decode_seqs": dseq, "decode_slots": dslot, "decode_positions": dpos,
                       "decode_share_groups": dgrp, "decode_share_rows": drows,
                       "prefill_slots": pslot, "prefill_positions": ppos, "copies": copies,
                       "chunks": chunks},
        }


# Rows a share group must save per launch, (members - 1) x shared rows, before
# its own launch pair pays: the prefix launch and the second decode cost about
# as much as reading 10-12k KV rows of 8 heads x 128 on MI355X.
SHARE_MIN_SAVED_ROWS = 24576


def decode_share_segments(groups, rows, min_members=2, min_saved_rows=SHARE_MIN_SAVED_ROWS):
    """Orders a decode batch by share group (Scheduler.step's decode_share_groups /
    decode_share_rows) for one attention launch per segment.

    A group qualifies with at least ``min_members`` entries this step whose
    shared rows are read ``(members - 1) * rows >= min_saved_rows`` fewer times
    when attended once (default SHARE_MIN_SAVED_ROWS: smaller groups run faster
    in the batch's plain launch; 0 sends every group of ``min_members`` through
    its own launch pair).

    Returns (order, segments): ``order`` permutes the decode entries so that
    entries without a qualifying group come first, then each group's entries
    together; ``segments`` lists
    (start, count, prefix_rows) over the permuted batch, prefix_rows 0 for the
    leading run (plain af_paged_attention) and the group's shared rows otherwise
    (af_paged_attention_shared_prefix with any member's table as the prefix).
    """
    groups = np.asarray(groups, np.int64)
    rows = np.asarray(rows, np.int32)
    if len(groups) != len(rows):
        raise ValueError("groups and rows differ in length")
    ids, counts = np.unique(groups[groups >= 0], return_counts=True)
    big = {}
    for g, c in zip(ids, counts):
        shared = np.unique(rows[groups == g])
        if len(shared) != 1:
            raise ValueError(f"group {g} has differing shared rows {shared.tolist()}")
        if c >= min_members and (c - 1) * int(shared[0]) >= min_saved_rows:
            big[int(g)] = int(shared[0])
    solo = [i for i, g in enumerate(groups) if int(g) not in big]
    order, segments = list(solo), []
    if solo:
        segments.append((0, len(solo), 0))
    for g in sorted(big):
        members = [i for i, x in enumerate(groups) if int(x) == g]
        segments.append((len(order), len(members), big[g]))
        order += members
    return np.array(order, np.int64), segments


def _nonneg(r, what):
    if r < 0:
        raise AfError(r, what)
    return r


__all__ = [
    "SHARE_MIN_SAVED_ROWS",
    "AF_KV_FP16", "AF_KV_FP8_E4M3", "AttentionWorkspace", "BlockManager", "build_rope_cache",
    "decode_share_segments", "default_splits", "fp8_quantize", "kv_copy_blocks", "launch_cached_attention",
    "launch_cached_attention_ex", "launch_decode_attention_fused", "launch_paged_attention",
    "launch_paged_decode_fused", "launch_paged_rope_append", "launch_qkv_rope_append",
    "launch_w8a16_gemv", "launch_prefill_rope_append", "launch_prefill_attention",
    "launch_tiled_attention_kernel", "launch_paged_prefill_attention", "Scheduler",
    "launch_paged_prefill_attention_batched", "prefill_tile_map",
    "launch_rope", "launch_rope_append", "launch_write_kv_cache", "make_pool", "paged_gather",
    "pool_bytes", "rope_table_host",
]
