/*
 * mlc_hip.h — C ABI of libmlc_hip.so, the MI355X runtime under mlc's HIP
 * backend. Plain pointers and sizes only; every function returns 0 on
 * success or a negative code (-hipError_t, or MLC_E_* below) and leaves a
 * message for mlc_last_error() on the calling thread.
 *
 * Each entry point replaces one piece of the reference's Triton/CUDA runtime
 * (paths relative to the reference repository):
 *
 *   mlc_ctx_create / mlc_ctx_destroy
 *       the per-model device state that mlc/runtime/executor.py:44-84
 *       (CompiledModel.__init__) sets up through torch.
 *   mlc_module_load / mlc_module_unload / mlc_function
 *       mlc/runtime/triton_runtime.py:47-65 (load_module + TritonRuntime):
 *       the generated kernels, as a gfx950 code object, and their handles.
 *   mlc_slab_alloc / mlc_slab_dlpack
 *       mlc/runtime/executor.py:158-162 (_get_arena, a torch.empty uint8
 *       arena) and :119-130 (_bind_arena): one hipMalloc slab, exported as a
 *       DLPack tensor so torch extern .out calls write into the same slab.
 *   mlc_launch
 *       mlc/runtime/triton_runtime.py:85-97 (TritonRuntime.launch) and
 *       mlc/runtime/executor.py:195-196 (fn[grid](*args, **consts)).
 *   mlc_plan_create / mlc_plan_set / mlc_plan_run / mlc_plan_destroy
 *       mlc/runtime/executor.py:165-202 (_build_plan / run_kernels): the
 *       pre-resolved launch sequence, run natively.
 *   mlc_graph_begin / mlc_graph_end / mlc_graph_replay
 *       mlc/runtime/executor.py:269-307 (_call_captured / _capture with
 *       torch.cuda.CUDAGraph): one captured hipGraph replayed per call.
 *   mlc_time_entry
 *       mlc/runtime/executor.py:309-352 (profile_kernels: CUDA-event timing of
 *       one plan entry in place), here with hipEvents on the launch stream.
 *   mlc_error_word / mlc_error_fetch / mlc_error_poll / mlc_error_clear
 *       the IndexError torch raises from aten.embedding for an id outside
 *       the table (mlc/runtime/executor.py:369-402 sends the op to torch):
 *       the native gather flags it in a device word instead, and the host
 *       reads the word's pinned mirror without stalling the stream.
 *   mlc_last_error
 *       the Python exceptions of the reference (ExecutionError etc.).
 */
#ifndef MLC_HIP_H
#define MLC_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MLC_OK 0
#define MLC_E_ARG (-10001)     /* invalid argument */
#define MLC_E_RANGE (-10002)   /* index or size out of range */
#define MLC_E_STATE (-10003)   /* call out of order (e.g. replay before capture) */

typedef struct mlc_ctx mlc_ctx;
typedef struct mlc_module mlc_module;
typedef struct mlc_plan mlc_plan;
typedef void* mlc_fn; /* a hipFunction_t */

/* Library version, (major << 16) | minor. */
int mlc_version(void);

/* Bind a context to HIP device `device` (made current on the calling thread). */
int mlc_ctx_create(int device, mlc_ctx** out);
int mlc_ctx_destroy(mlc_ctx* ctx);

/* Load a gfx950 code object image (hipModuleLoadData) / look up a kernel. */
int mlc_module_load(mlc_ctx* ctx, const void* image, size_t size, mlc_module** out);
int mlc_module_unload(mlc_module* mod);
int mlc_function(mlc_module* mod, const char* name, mlc_fn* out);

/* The arena: one hipMalloc of at least `bytes` (grown, never shrunk, while
 * no export is alive). Offsets the planner assigns are byte offsets into it. */
int mlc_slab_alloc(mlc_ctx* ctx, size_t bytes, void** dptr);
/* A DLManagedTensor* (uint8, 1-D, the whole slab, kDLROCM) for torch's
 * from_dlpack; its deleter releases one reference on the slab. */
int mlc_slab_dlpack(mlc_ctx* ctx, void** managed_tensor);

/* The arena for callers that cannot allocate (code under graph capture,
 * serving loops, harnesses that forbid hipMalloc). It has no counterpart in
 * the reference: a variant of mlc_slab_alloc that allocates nothing. The
 * context's arena becomes the library's static device array of
 * MLC_STATIC_SLAB_BYTES (one per GPU, 256-B aligned, held from the first
 * context on that GPU until the process ends; its address is resolved once
 * per device in mlc_ctx_create). Returns MLC_E_RANGE for `bytes` beyond the
 * maximum and MLC_E_STATE if the context already holds an allocated slab.
 * Calls no hipMalloc, hipFree or other allocating routine. Every context on
 * one GPU that uses it shares the one array, which keeps the last run's
 * contents (the planner writes every arena buffer before reading it, so
 * nothing needs clearing): runs that overlap on one GPU race. */
#define MLC_STATIC_SLAB_BYTES (64u << 20)
int mlc_slab_static(mlc_ctx* ctx, size_t bytes, void** dptr);

/* Launch one kernel; `kernarg` holds `size` bytes of packed arguments. */
int mlc_launch(mlc_fn fn, uint32_t grid, uint32_t block, uint32_t lds_bytes,
               const void* kernarg, size_t size, void* stream);

/* A pre-resolved sequence of launches. */
int mlc_plan_create(mlc_ctx* ctx, int n_entries, mlc_plan** out);
int mlc_plan_set(mlc_plan* plan, int index, mlc_fn fn, uint32_t grid, uint32_t block,
                 uint32_t lds_bytes, const void* kernarg, size_t size);
/* Launch entries [begin, end) in order on `stream`. */
int mlc_plan_run(mlc_plan* plan, int begin, int end, void* stream);
int mlc_plan_destroy(mlc_plan* plan);

/* Stream capture into the context's graph (thread-local capture mode). */
int mlc_graph_begin(mlc_ctx* ctx, void* stream);
int mlc_graph_end(mlc_ctx* ctx);
int mlc_graph_replay(mlc_ctx* ctx, void* stream);
/* Number of nodes in the captured graph (for checks), or negative. */
int mlc_graph_node_count(mlc_ctx* ctx, size_t* out);

/* Average milliseconds of `iters` back-to-back launches of plan entry `index`
 * on `stream`, measured with hipEvents recorded on that stream. */
int mlc_time_entry(mlc_plan* plan, int index, int iters, void* stream, float* ms_out);

/* The context's invalid-input word (16 bytes of device memory, zeroed when
 * first requested, with a pinned host mirror). Kernels that meet an invalid
 * input (an embedding id outside its table) store a non-zero value in it. */
int mlc_error_word(mlc_ctx* ctx, void** device_word);
/* Enqueue an asynchronous copy of the word to its host mirror on `stream`
 * (may be captured into a graph). */
int mlc_error_fetch(mlc_ctx* ctx, void* stream);
/* The host mirror's first int as of the last completed fetch; no sync. */
int mlc_error_poll(mlc_ctx* ctx, int32_t* value);
/* Synchronize the device, then zero the word and its mirror. */
int mlc_error_clear(mlc_ctx* ctx);

/* Synchronize the context's device. */
int mlc_device_synchronize(mlc_ctx* ctx);

/* Message of the last failure on this thread ("" if none). */
const char* mlc_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* MLC_HIP_H */
