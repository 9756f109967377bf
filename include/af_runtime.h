/*
 * af_runtime.h — device plumbing exported by libatomflow_kv.so.
 *
 * No counterpart in the reference: AtomFlow calls the CUDA runtime directly
 * from C++ (cudaMalloc, cudaStreamCreate, cudaEvent*, graph capture in
 * src/main.cu:92-150). These thin wrappers let an FFI host (ctypes, cgo, JNI)
 * drive the KV path without a second GPU runtime in the process. Same status
 * convention as af_kv.h.
 */
#ifndef AF_RUNTIME_H_
#define AF_RUNTIME_H_

#include <stddef.h>
#include <stdint.h>

#include "af_kv.h"

#ifdef __cplusplus
extern "C" {
#endif

int af_rt_device_count(int* count);
int af_rt_set_device(int device);
/* Name, compute units and gfx arch of the current device. */
int af_rt_device_info(char* name, int name_len, int* compute_units, char* arch, int arch_len);
int af_rt_device_sync(void);
/* Returns and clears the runtime's sticky last error. */
int af_rt_last_error(void);

int af_rt_malloc(void** ptr, size_t bytes);
int af_rt_free(void* ptr);
int af_rt_host_malloc(void** ptr, size_t bytes); /* pinned */
int af_rt_host_free(void* ptr);
int af_rt_mem_info(size_t* free_bytes, size_t* total_bytes);

/* Copies are ordered on `stream`; the *_sync forms wait for completion. */
int af_rt_memcpy_h2d(void* dst, const void* src, size_t bytes, af_stream_t stream);
int af_rt_memcpy_d2h(void* dst, const void* src, size_t bytes, af_stream_t stream);
int af_rt_memcpy_d2d(void* dst, const void* src, size_t bytes, af_stream_t stream);
/* Fill with a 32-bit pattern (a kernel, safe inside stream capture). */
int af_rt_fill_u32(void* dst, uint32_t value, size_t n_words, af_stream_t stream);
/* d_values[i] += delta for i < n (a kernel: a captured decode step uses it to
 * advance its device-resident position and length). */
int af_rt_add_i32(int32_t* d_values, int n, int32_t delta, af_stream_t stream);
/* Synthetic N(0,1) fp16 data on the device: counter-based hash + Box-Muller.
 * Deterministic in (seed, index); for bench-scale inputs only. */
int af_rt_fill_randn_f16(void* dst, size_t n, uint64_t seed, float stddev, af_stream_t stream);
/* Synthetic FP8 E4M3 codes of N(0,1)/scale values (bench-scale inputs). */
int af_rt_fill_randn_fp8(uint8_t* dst, size_t n, uint64_t seed, float inv_scale, af_stream_t stream);

/* Streaming-read probe, a measurement aid: reads `bytes` at src once (16-B
 * loads, no compute) and writes at most one word of d_sink. segment_bytes 0:
 * `workgroups` contiguous chunks (the read ceiling for a launch of this size).
 * segment_bytes 256 (fp16) or 128 (FP8): the decode-attention kernel's access
 * pattern for head_dim 128 without its arithmetic. src holds two equal slabs
 * (K then V) of rows of row_bytes; workgroups = splits x (row_bytes /
 * segment_bytes), each reading one head segment of one split's rows.
 * nontemporal != 0: the loads use the non-temporal (streaming) cache policy, as
 * the decode kernels' KV row loads do. */
int af_rt_read_probe(const void* src, size_t bytes, int workgroups, int segment_bytes,
                     int row_bytes, int nontemporal, uint32_t* d_sink, af_stream_t stream);

int af_rt_stream_create(af_stream_t* stream);
int af_rt_stream_destroy(af_stream_t stream);
int af_rt_stream_sync(af_stream_t stream);

int af_rt_event_create(void** event);
int af_rt_event_destroy(void* event);
int af_rt_event_record(void* event, af_stream_t stream);
int af_rt_event_sync(void* event);
int af_rt_event_elapsed_ms(float* ms, void* start, void* stop);

/* Stream capture into a hipGraph and replay. */
int af_rt_capture_begin(af_stream_t stream);
int af_rt_capture_end(af_stream_t stream, void** graph_exec);
int af_rt_graph_launch(void* graph_exec, af_stream_t stream);
int af_rt_graph_destroy(void* graph_exec);

#ifdef __cplusplus
}
#endif
#endif /* AF_RUNTIME_H_ */
