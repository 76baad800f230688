/*
 * libtforge_hip -- C ABI of the MI355X (gfx950) backend for TensorForge's GPU
 * hot path: the fused fp32 relu(A @ B + bias) kernel, plain matmul, and the
 * bias_add / relu / add epilogues that --tforge-gpu-pipeline emits.
 *
 * The reference crosses three boundaries on this path (paths in the
 * TensorForge tree); this library replaces all three in one process:
 *   1. compile:  tensorforge-opt --tforge-gpu-pipeline="<opts>" + the NVVM/ptxas
 *                chain (python/tforge_gpu.py:66-91)          -> tf_compile
 *   2. kernel ABI: one noalias device pointer per entry argument, then the
 *                result out-param (runners/gpu/tforge-gpu-bench.cu:20-24;
 *                lib/Transforms/Gpu.cpp:494-512, 563-570)   -> tf_launch
 *   3. runner:   tforge-gpu-bench --mode kernel|cublas [--info-only]
 *                (runners/gpu/tforge-gpu-bench.cu:92-140, 175-383)
 *                                                           -> tf_run, tf_bench,
 *                                                              tf_kernel_info
 *
 * Conventions: plain pointers and sizes only.  Every int-returning function
 * returns 0 on success or a negative TF_E* code, and tf_last_error() then
 * holds the message (the reference printed it and exited 1:
 * runners/gpu/tforge-gpu-bench.cu:52-70; the Python wrapper raises
 * RuntimeError with it, python/tforge_cpu.py:216-222).  Handles are not shared
 * between threads.  All tensors are row-major float32.
 */
#ifndef TFORGE_HIP_H
#define TFORGE_HIP_H

#ifdef __cplusplus
extern "C" {
#endif

#define TF_OK 0
#define TF_E_PARSE -1    /* program text does not parse or verify            */
#define TF_E_OPTIONS -2  /* malformed pipeline option string                 */
#define TF_E_PLAN -3     /* program/option combination the pipeline rejects */
#define TF_E_ARG -4      /* bad argument to an API call                       */
#define TF_E_HIP -5      /* HIP runtime error                                 */
#define TF_E_BLAS -6     /* vendor BLAS baseline unavailable or failed        */

#define TF_FAMILY_DIRECT 0      /* tile-k=0: one FMA chain per output          */
#define TF_FAMILY_STAGED 1      /* tile-k>0: LDS-staged FP32 MFMA              */
#define TF_FAMILY_ELEMENTWISE 2 /* programs without a matmul                   */
#define TF_FAMILY_WAVEK 4       /* tile-k>0 with wave-split-k: the waves of a
                                   workgroup split K, partial tiles summed in
                                   LDS (one launch, no workspace)              */

#define TF_MODE_KERNEL 0 /* the compiled program                            */
#define TF_MODE_BLAS 1   /* rocBLAS sgemm + a separate epilogue kernel: the
                            counterpart of the reference's --mode cublas
                            (runners/gpu/tforge-gpu-bench.cu:303-318)       */

typedef struct tf_kernel tf_kernel_t; /* opaque: one compiled tforge program */

/* Device facts; replaces the runner's cuDeviceGetName/driver queries
 * (runners/gpu/tforge-gpu-bench.cu:180-186, 367-368). */
typedef struct {
  char name[256];
  char arch[64];
  int compute_units;
  int max_clock_mhz;
  int lds_bytes_per_cu;
  int max_threads_per_cu;
  long long l2_bytes;
  long long global_mem_bytes;
  int driver_version;
  int runtime_version;
} tf_device_info_t;

/* Static launch description of one kernel of a compiled program; replaces
 * the tforge.launch attribute / launch.json (lib/Transforms/Gpu.cpp:572-577,
 * python/tforge_gpu.py:42-51, 88-90). */
typedef struct {
  char kernel[96];   /* instantiation name                                   */
  char args[160];    /* buffer order, reference "argN" spelling              */
  char ops[96];      /* fused ops of this launch, e.g. matmul+bias_add+relu  */
  int family;        /* TF_FAMILY_*                                          */
  int grid[3];
  int block[3];
  long long m, n, k; /* problem of this launch (k = 0 for element ops)       */
  int lds_bytes;     /* static LDS of the instantiation                      */
} tf_launch_info_t;

/* Resources and occupancy of one kernel; replaces --info-only
 * (runners/gpu/tforge-gpu-bench.cu:278-291).  Needs a GPU. */
typedef struct {
  int regs;          /* VGPRs per lane as reported by hipFuncGetAttributes   */
  int local_bytes;   /* private (scratch) bytes per lane                     */
  int static_smem;   /* static LDS bytes per workgroup                       */
  int blocks_per_cu; /* hipOccupancyMaxActiveBlocksPerMultiprocessor         */
  double theo_occupancy; /* resident waves / max waves per CU                */
  int threads;
} tf_kernel_resources_t;

/* One buffer of the program's kernel ABI (argN order: entry arguments, then
 * the result). */
typedef struct {
  char name[64];
  int role;          /* 0 input, 1 output                                     */
  long long rows, cols; /* 2-D view: leading dims flattened into rows         */
} tf_buffer_info_t;

/* Timing of tf_bench; replaces the runner's JSON line
 * (runners/gpu/tforge-gpu-bench.cu:363-381). */
typedef struct {
  double median_ms, min_ms, mean_ms, std_ms;
  double clock_median_mhz, clock_min_mhz, clock_max_mhz;
  double power_median_w;
  int warmup, reps, l2_flush;
  long long padded[3]; /* problem the kernel ran at (Mp, Np, Kp)             */
} tf_bench_result_t;

const char *tf_last_error(void);

/* Device 0 facts (the reference runner also uses device 0 and reports its
 * name and driver in the JSON line, runners/gpu/tforge-gpu-bench.cu:367-381). */
int tf_device_info(tf_device_info_t *out);

/* Parse + verify `program` (tforge text, diagnostics name `source_name`),
 * parse `options` (--tforge-gpu-pipeline option string, may be empty), plan the
 * launches and select the gfx950 instantiations.  No GPU work: runs on a host
 * without a GPU.  Replaces python/tforge_gpu.py:66-91 (compile_kernel's
 * tool chain).  Options are the reference's (include/TensorForge/Pipelines.h:45-72)
 * plus four backend options: split-k=S (S workgroups per output tile along K,
 * then an ordered reduction launch), mask-edges (staged kernels accept shapes
 * that are not tile multiples), wave-split-k (each wave of a workgroup
 * reduces its own K range of the workgroup's tile, the partial tiles are
 * added in LDS in wave order: one launch for shapes with few output tiles)
 * and xcd-swizzle (default on).
 * Staged configurations (tile-k > 0) give each 64-lane wave an
 * (8*TM) x (8*TN) output tile of MFMA blocks.  Where that wave tile cannot
 * tile the block -- fewer than 64 threads, or a wave tile taller or wider
 * than the block tile, as in 30 of the reference's 105 Stage 9
 * configurations (python/costmodel.py:49-60) -- the same block tile and
 * tile-k run on a stand-in wave layout: one wave over the whole block when
 * there are fewer than 64 threads (thread tile BM/8 x BN/8), otherwise the
 * same threads and accumulators per lane with the long side of the thread
 * tile shortened to fit.  tf_kernel_launch_info then reports the block
 * actually launched and the instantiation's name. */
int tf_compile(const char *source_name, const char *program, const char *options, tf_kernel_t **out);
void tf_kernel_free(tf_kernel_t *k);

/* The compiled program's launches (one, or two for the residual block) and
 * buffers: what the reference reads back from launch.json and the runner's
 * --grid/--block/--args flags (python/tforge_gpu.py:42-51, 88-90;
 * runners/gpu/tforge-gpu-bench.cu:20-24, 92-140). */
int tf_kernel_num_launches(const tf_kernel_t *k);
int tf_kernel_launch_info(const tf_kernel_t *k, int launch, tf_launch_info_t *out);
int tf_kernel_num_buffers(const tf_kernel_t *k); /* entry arguments + 1 result */
int tf_kernel_buffer_info(const tf_kernel_t *k, int index, tf_buffer_info_t *out);
/* Shape (rows x cols) of buffer `index` as tf_run / tf_bench copy it from and
 * to host memory: the compiled shape, or, with `logical_mnk`, the logical
 * shape of the buffer's role in the single matmul chain (A m x k, B k x n,
 * bias 1 x n, residual and result m x n; an unused argument keeps its compiled
 * shape).  Fails with TF_E_ARG where tf_run would refuse the logical sizes (a
 * multi-launch program, sizes above the compiled ones, or one buffer in two
 * roles whose logical shapes differ).  The counterpart of the reference
 * runner's per-buffer --in-dir file sizes (runners/gpu/tforge-gpu-bench.cu:214-232). */
int tf_kernel_host_shape(const tf_kernel_t *k, const long long *logical_mnk, int index, long long *rows,
                         long long *cols);
/* Resources and occupancy of one launch: the runner's --info-only
 * (runners/gpu/tforge-gpu-bench.cu:278-291). */
int tf_kernel_info(const tf_kernel_t *k, int launch, tf_kernel_resources_t *out);

/* Kernel ABI: enqueue every launch of the program on `stream` (a hipStream_t,
 * NULL for the default stream) with caller-owned device buffers in argN order,
 * shaped as compiled: tf_kernel_num_buffers(k) pointers, the inputs then the
 * result, each to the float32 elements tf_kernel_buffer_info reports.  A NULL
 * pointer for a non-empty buffer is refused (TF_E_ARG) before any launch.
 * Intermediates of multi-launch programs and the split-K
 * partial-sum workspace are allocated once per handle on first use; calls on
 * one handle that overlap on different streams share them.  No
 * synchronisation.  Replaces cuLaunchKernel with the marshalled argN list
 * (runners/gpu/tforge-gpu-bench.cu:259-299). */
int tf_launch(tf_kernel_t *k, void *const *device_buffers, void *stream);

/* tf_launch without any device allocation, for callers that cannot allocate
 * (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  Same arguments and kernels as
 * tf_launch; the split-K workspace and the intermediates of multi-launch
 * programs come from one fixed 32 MiB device array per GPU (held from the
 * library's first use on that GPU until the process ends) instead of the
 * handle's buffers.  A program that needs more scratch than that is refused
 * with TF_E_ARG before anything is enqueued.  Nothing in the array needs
 * clearing between calls (every slice and intermediate is written whole
 * before it is read), but every call on one GPU shares it: calls that overlap
 * on that GPU -- from any handle or stream -- race, so serialise them.
 * `stream` must belong to the current device (TF_E_ARG otherwise).  The
 * array's device address is looked up on the first call on each device; that
 * first call may itself be under stream capture. */
int tf_launch_noalloc(tf_kernel_t *k, void *const *device_buffers, void *stream);

/* Correctness run, as the runner's "--warmup 0 --reps 1 --in-dir --out":
 * uploads host inputs, NaN-prefills the output, runs once, downloads the
 * result.  `logical_mnk` (may be NULL) gives the unpadded M, N, K of a
 * single-matmul program compiled at a padded shape: inputs and output are then
 * at the logical shape and the library pads and unpads with device copies,
 * as the reference runner does (runners/gpu/tforge-gpu-bench.cu:214-232,
 * 292-302, 323-331).  host_inputs holds one row-major float32 array per
 * input, each of the size tf_kernel_host_shape reports for the same
 * `logical_mnk` (M x K, K x N and N elements for A, B and bias at a logical
 * shape; the compiled shapes otherwise), and host_out has room for the result;
 * the library copies exactly those sizes.  mode is TF_MODE_KERNEL or TF_MODE_BLAS. */
int tf_run(tf_kernel_t *k, int mode, const long long *logical_mnk, const float *const *host_inputs,
           float *host_out);

/* Timing run: inputs from `host_inputs` (or, if NULL, uniform[-1,1] from
 * `seed`), `warmup` untimed runs, then `reps` runs each bracketed by a HIP
 * event pair on the library's stream (pad copies included when padded, an
 * optional 512 MiB L2/MALL flush before each rep outside the events), the
 * shader clock (tf_clock_probe) and, where amdsmi loads, the power sampled
 * after each rep.  Replaces
 * runners/gpu/tforge-gpu-bench.cu:337-381. */
int tf_bench(tf_kernel_t *k, int mode, const long long *logical_mnk, const float *const *host_inputs,
             unsigned seed, int warmup, int reps, int flush, tf_bench_result_t *out);

/* Shader clock (MHz) measured on the device: a probe kernel after the work
 * already queued on `stream` (a hipStream_t, NULL for the default stream)
 * counts shader-clock cycles against the 100 MHz wall clock in one workgroup
 * per XCD; mean, min and max over the XCDs (min/max may be NULL).
 * Synchronises the stream.  Each call writes its own result slot (64 slots
 * per GPU, taken round robin), so calls from several threads or streams may
 * overlap.  tf_bench takes one such sample after every rep;
 * the reference samples the SM clock through NVML instead
 * (runners/gpu/tforge-gpu-bench.cu:333-361). */
int tf_clock_probe(void *stream, double *mean_mhz, double *min_mhz, double *max_mhz);

/* Per-rep event times (ms) of the last tf_bench on this handle, up to `cap`
 * values; returns the count.  No counterpart in the reference (its runner
 * prints only median/min/std); for callers that want the distribution. */
int tf_bench_samples(const tf_kernel_t *k, double *out_ms, int cap);

/* Registry introspection: number of ahead-of-time instantiations and the
 * staged configuration of entry i (family, bm, bn, tm, tn, bk, promote,
 * vectorize) -- what the autotuner may select.  No counterpart in the
 * reference, which generates each kernel on demand. */
int tf_registry_size(void);
int tf_registry_entry(int i, int *family, int *cfg7, char *name, int name_cap);

#ifdef __cplusplus
}
#endif

#endif /* TFORGE_HIP_H */
