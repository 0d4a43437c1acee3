/*
 * shlo_hip.h — the C ABI of the MI355X StableHLO executor (libshlo_hip.so).
 *
 * This is the drop-in replacement for the reference's FFI boundary,
 * c/smlx_shim.c, which StablehloMlx/Mlx.lean:16-73 binds with 25 @[extern]
 * declarations.  Each shlo_* entry point below replaces the smlx_* function
 * named beside it (file:line in the reference) one to one: same arguments,
 * same meaning, same error behaviour, with plain C types in place of Lean
 * objects:
 *
 *   - arrays, kernels and traced functions are opaque handles; every handle a
 *     call returns is owned by the caller and released with its *_free
 *     function (the Lean finalizers of c/smlx_shim.c:45-58, :277-281, :327-331);
 *   - every call returns 0 on success or nonzero on failure, and
 *     shlo_last_error() then returns the "what: detail" message for this
 *     thread (the IO user errors of c/smlx_shim.c:15-41);
 *   - shapes are int64 arrays with rank <= 16 (c/smlx_shim.c:60-65), row-major;
 *   - dtype codes are the mlx_dtype enum order the reference uses
 *     (StablehloMlx/Mlx.lean:28-37): bool 0, u8 1, u16 2, u32 3, u64 4, i8 5,
 *     i16 6, i32 7, i64 8, f16 9, f32 10; this library adds f64 11.
 *
 * Arrays live in the GPU's HBM and stay there between calls; only
 * shlo_to_bytes copies to the host.  Work is ordered on one HIP stream and
 * runs asynchronously; shlo_eval waits for it.  Not thread-safe (like the
 * reference shim, c/smlx_shim.c:21-28).
 *
 * Beyond the 25, the executor surface of StablehloMlx/Exec.lean and a few
 * measurement helpers are exported at the end (marked as such).
 */
#ifndef SHLO_HIP_H
#define SHLO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct shlo_arr shlo_arr;
typedef struct shlo_kernel shlo_kernel;
typedef struct shlo_fn shlo_fn;

/* The last error message of this thread ("" if none). */
const char *shlo_last_error(void);

/* Release an array handle (Arr finalizer, c/smlx_shim.c:45-48). NULL is a no-op. */
void shlo_arr_free(shlo_arr *a);

/* ---- construction and readback ------------------------------------------- */

/* smlx_empty (c/smlx_shim.c:87-90): an empty array (f32, shape [0]). */
int shlo_empty(shlo_arr **out);

/* smlx_of_bytes (c/smlx_shim.c:92-103): a new array holding `nbytes` bytes of
 * raw little-endian row-major elements; nbytes must equal count*dtype size. */
int shlo_of_bytes(const void *data, size_t nbytes, const int64_t *shape, size_t rank, uint8_t dtype,
                  shlo_arr **out);

/* smlx_to_bytes (c/smlx_shim.c:105-127): waits for the array, then copies it
 * out row-major (a strided view reads back in logical order).  With dst NULL
 * only *nbytes is set; otherwise cap must be >= the array's byte size. */
int shlo_to_bytes(const shlo_arr *a, void *dst, size_t cap, size_t *nbytes);

/* smlx_shape (c/smlx_shim.c:129-136): writes up to cap dims, sets *rank. */
int shlo_shape(const shlo_arr *a, int64_t *shape, size_t cap, size_t *rank);

/* smlx_dtype (c/smlx_shim.c:138-140). */
int shlo_dtype(const shlo_arr *a, uint8_t *dtype);

/* ---- ops: one executor op each -------------------------------------------- */

/* smlx_unary (c/smlx_shim.c:148-166); op codes of StablehloMlx/Mlx.lean:76-87:
 * neg 0, abs 1, sqrt 2, floor 3, exp 4, erf 5, not 6, invert 7, rsqrt 8,
 * tanh 9, sigmoid 10. */
int shlo_unary(uint32_t op, const shlo_arr *a, shlo_arr **out);

/* smlx_binary (c/smlx_shim.c:168-196); op codes of StablehloMlx/Mlx.lean:88-108:
 * add 0, sub 1, mul 2, div 3, max 4, min 5, and 6, or 7, xor 8, shl 9, shr 10,
 * eq 11, ne 12, lt 13, le 14, gt 15, ge 16, matmul 17, rem 18, land 19, lor 20.
 * Operands broadcast (numpy rules). */
int shlo_binary(uint32_t op, const shlo_arr *a, const shlo_arr *b, shlo_arr **out);

/* smlx_where (c/smlx_shim.c:198-201). */
int shlo_where(const shlo_arr *c, const shlo_arr *a, const shlo_arr *b, shlo_arr **out);
/* smlx_reshape (c/smlx_shim.c:203-208). */
int shlo_reshape(const shlo_arr *a, const int64_t *shape, size_t rank, shlo_arr **out);
/* smlx_transpose (c/smlx_shim.c:210-215). */
int shlo_transpose(const shlo_arr *a, const int64_t *perm, size_t n, shlo_arr **out);
/* smlx_broadcast (c/smlx_shim.c:217-222). */
int shlo_broadcast(const shlo_arr *a, const int64_t *shape, size_t rank, shlo_arr **out);
/* smlx_slice (c/smlx_shim.c:224-229). */
int shlo_slice(const shlo_arr *a, const int64_t *start, const int64_t *stop, const int64_t *step, size_t n,
               shlo_arr **out);
/* smlx_concat (c/smlx_shim.c:231-239). */
int shlo_concat(const shlo_arr *const *xs, size_t n, uint32_t axis, shlo_arr **out);
/* smlx_astype (c/smlx_shim.c:241-244). */
int shlo_astype(const shlo_arr *a, uint8_t dtype, shlo_arr **out);
/* smlx_view (c/smlx_shim.c:246-249): reinterpret the bytes as another dtype. */
int shlo_view(const shlo_arr *a, uint8_t dtype, shlo_arr **out);
/* smlx_take (c/smlx_shim.c:251-254): indices are clamped to the axis. */
int shlo_take(const shlo_arr *a, const shlo_arr *idx, uint32_t axis, shlo_arr **out);
/* smlx_max_axis (c/smlx_shim.c:256-259): the axis is removed. */
int shlo_max_axis(const shlo_arr *a, uint32_t axis, shlo_arr **out);
/* smlx_contiguous (c/smlx_shim.c:261-264). */
int shlo_contiguous(const shlo_arr *a, shlo_arr **out);
/* smlx_eval (c/smlx_shim.c:266-273): wait until the arrays are computed. */
int shlo_eval(const shlo_arr *const *xs, size_t n);

/* ---- precompiled kernels (replacing mx::fast::metal_kernel) --------------- */

/* smlx_kernel_new (c/smlx_shim.c:283-297): resolve `name` ("mul_mat",
 * "soft_max", "norm", "silu", "gelu_erf", "erff_map", "expf_map", "divide", "sqrt",
 * "f64_ew", "f64_of_f32", "f32_of_f64"; an "smlx_" prefix is accepted) to a
 * precompiled gfx950 kernel.  The binding names, source and header of the
 * reference's Metal spec are accepted and ignored (nothing is compiled at run
 * time).  Unknown names fail. */
int shlo_kernel_new(const char *name, const char *const *inputs, size_t nin, const char *const *outputs,
                    size_t nout, const char *source, const char *header, shlo_kernel **out);
void shlo_kernel_free(shlo_kernel *k);

/* smlx_kernel_apply (c/smlx_shim.c:299-323): inputs in the kernel's binding
 * order, the last one being the u32 parameter array of
 * StablehloMlx/Kernels/Run.lean:64-104 (e.g. mul_mat: [K, M, R,
 * wBatchStride, N, plain]).  out_shapes holds the nout output shapes
 * back to back (out_ranks[i] dims each); grid and threadgroup are accepted
 * and checked for 3 entries, and the kernel picks its own launch shape.
 * outs receives nout new arrays. */
int shlo_kernel_apply(const shlo_kernel *k, const shlo_arr *const *inputs, size_t nin, const int64_t *out_shapes,
                      const size_t *out_ranks, const uint8_t *out_dtypes, size_t nout, const int64_t *grid,
                      size_t grid_n, const int64_t *threadgroup, size_t tg_n, shlo_arr **outs);

/* ---- compiled functions (replacing mx::compile) ----------------------------- */

/* The traced host function: given nin input arrays, it returns up to out_cap
 * new arrays in outputs[] (owned by the caller of the callback) and their
 * count in *nout; it returns 0, or nonzero after shlo_set_error(). */
typedef int (*shlo_traced_fn)(void *payload, const shlo_arr *const *inputs, size_t nin, shlo_arr **outputs,
                              size_t out_cap, size_t *nout);

/* smlx_compile (c/smlx_shim.c:359-374): wrap `fn`.  With enable != 0 the first
 * apply for each input signature traces `fn` (its ops are recorded, not run)
 * and captures the recorded launches into a hipGraph (traces shorter than
 * shlo_set_graph_min_ops' threshold keep the recorded launches instead); every
 * apply then copies the inputs into the trace's input buffers (skipped when
 * the same array is passed again), launches the graph (or re-issues the
 * launches) and returns fresh output arrays.  With enable == 0 every apply
 * calls `fn` eagerly.
 * payload_free (may be NULL) is called on payload when the fn is freed. */
int shlo_compile(shlo_traced_fn fn, void *payload, void (*payload_free)(void *), int enable, shlo_fn **out);
void shlo_fn_free(shlo_fn *f);

/* smlx_apply (c/smlx_shim.c:376-386). */
int shlo_apply(shlo_fn *f, const shlo_arr *const *inputs, size_t nin, shlo_arr **outs, size_t out_cap,
               size_t *nout);

/* Set this thread's error message (for traced callbacks reporting failure,
 * the trace_error of c/smlx_shim.c:30-41). */
void shlo_set_error(const char *msg);

/* ---- test-driver helpers ---------------------------------------------------- */

/* smlx_libm_erff_range (c/smlx_shim.c:388-403): the executor's erff (the
 * correctly rounded routine its kernels run, evaluated on the host) over
 * count consecutive binary32 bit patterns from base, as bit patterns. */
int shlo_libm_erff_range(uint32_t base, uint32_t count, uint32_t *out);

/* smlx_count_nonzero (c/smlx_shim.c:405-414). */
int shlo_count_nonzero(const shlo_arr *a, uint64_t *out);

/* ==== Beyond the reference shim ============================================== */

/* The executor surface of StablehloMlx/Exec.lean:17-43 and Lower.lean's
 * planted faults (one bit per field of Lower.Faults, Lower.lean:53-69, in
 * declaration order: dotBuiltin 0, dotPlain 1, softMaxFloatSum 2, normGpuOps 3,
 * siluGpuOps 4, geluTanh 5, divideBuiltin 6, sqrtBuiltin 7, binaryHalf 8,
 * broadcastFirst 9, concatSwap 10, transposeIdentity 11, sliceShift 12,
 * f64AsF32 13, whileShort 14). */
typedef struct shlo_module shlo_module;
/* Exec.load (Exec.lean:21-27): parse; the module must have @main. */
int shlo_module_load(const char *text, size_t len, shlo_module **out);
void shlo_module_free(shlo_module *m);
/* Exec.argTys (Exec.lean:40): @main's argument count and types (element type
 * as its dtype code). */
int shlo_module_nargs(const shlo_module *m, size_t *n);
int shlo_module_arg(const shlo_module *m, size_t i, int64_t *shape, size_t cap, size_t *rank, uint8_t *dtype);
/* Exec.prepare (Exec.lean:30-31): the module's @main as a (compiled) fn. */
int shlo_module_prepare(const shlo_module *m, uint64_t faults, int compile, shlo_fn **out);
/* Exec.call (Exec.lean:34-37): apply and wait. */
int shlo_call(shlo_fn *f, const shlo_arr *const *inputs, size_t nin, shlo_arr **outs, size_t out_cap,
              size_t *nout);

/* The ggml_vec_dot_f32 tail flavour used by dot_general: 0 stock (the
 * reference's mul_mat kernel, Shaders.lean:80-90), 1 pinned (unfused tail). */
int shlo_set_flavor(int flavor);
int shlo_get_flavor(void);

/* Compiled functions (shlo_compile, shlo_module_prepare with compile = 1)
 * whose trace holds at least n recorded launches are captured into one
 * hipGraph; shorter traces re-issue their recorded launches on the stream
 * (same kernels, same buffers, same bits).  Takes effect for functions traced
 * afterwards (a function is traced on its first call per input signature).
 * Default 32 (or the environment's SHLO_GRAPH_MIN_OPS); n = 1 captures every
 * trace.  *prev receives the old value when prev is not NULL.  Not in the
 * reference (mlx compiles to its own graph). */
int shlo_set_graph_min_ops(int n, int *prev);

/* The correctly rounded expf that ggml's scalar row tails use in the pinned
 * flavour (soft_max and silu rows with cols % 4 != 0; the stock flavour
 * refuses them, as the reference does), evaluated on the host over count
 * consecutive binary32 bit patterns from base, as bit patterns: the CPU side
 * of its exhaustive check.  The GPU side is the precompiled kernel "expf_map"
 * (inputs [u32 params: base, count], one u32 output of count words).  Not in
 * the reference. */
int shlo_expf_range(uint32_t base, uint32_t count, uint32_t *out);

/* Measurement helpers (not in the reference): a device-side fill from the
 * splitmix32 stream of ref/ggml_ref.c:21-30 — dist 0: unif(a) with a =
 * param (ggml_ref.c:30), element i using draw i; dist 1: the Irwin-Hall
 * normal (sum of 12 draws' top 24 bits * 2^-24, minus 6, times sigma = param,
 * one rounding), element i using draws 12i..12i+11.  The stream starts at
 * `seed` and skips `skip` draws first. */
int shlo_fill_random(const int64_t *shape, size_t rank, uint32_t seed, uint64_t skip, int dist, double param,
                     shlo_arr **out);
/* The order-free checksum of 32-bit words used by the exhaustive erff fixture:
 * sum over t of (w[t]+1)*(2(start+t)+1)*0x9E3779B97F4A7C15 mod 2^64. */
int shlo_checksum_u32(const shlo_arr *a, uint64_t start_index, uint64_t *out);
/* Wait for all queued work. */
int shlo_sync(void);
/* hipEvent timing on the executor's stream: start records an event, stop
 * records another, waits, and returns the milliseconds between them. */
int shlo_timer_start(void);
int shlo_timer_stop(float *ms);
/* Apply `f` to the same inputs `reps` times back to back (outputs dropped at
 * once) between two HIP events on the executor's stream; *ms = the mean
 * milliseconds per apply.  Host call overhead stays outside the timed loop. */
int shlo_time_apply(shlo_fn *f, const shlo_arr *const *inputs, size_t nin, int reps, float *ms);
/* Device name, compute units and the bytes the array pool holds. */
int shlo_device_info(char *name, size_t cap, int *cus, uint64_t *pool_bytes);
/* No counterpart in the reference.  shlo_count_nonzero for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc): counts the elements among `count`
 * elements of elem_bytes (1, 2, 4 or 8) bytes at device address `data` whose
 * bytes are not all zero, and writes the count to the device word
 * `out_device`.  The work is queued on the executor's stream (shlo_sync
 * waits for it).  Partial counts live in a static device array of 4096 words
 * (32 KiB per GPU, held until the process ends), so the call allocates and
 * frees nothing; at most 2^40 elements per call.  Both ranges must lie inside
 * device allocations (checked; an error otherwise).  Calls that overlap on
 * one GPU from different streams or processes race on the shared array. */
int shlo_count_nonzero_noalloc(const void *data, uint64_t count, uint32_t elem_bytes, uint64_t *out_device);
/* The kernel family and template arguments that the most recent dot_general
 * (or mul_mat) dispatch chose, e.g. "dot_mfma8d_k<RowVecB,ColQuadB,128,8>",
 * written NUL-terminated into name[cap] ("" before the first dispatch).  Lets
 * tests check that a shape reaches the kernel it is meant to exercise. */
int shlo_last_dot_kernel(char *name, size_t cap);
/* The device address of an array's first element (for in-place interop). */
int shlo_data_ptr(const shlo_arr *a, void **ptr);

#ifdef __cplusplus
}
#endif
#endif
