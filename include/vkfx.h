/*
 * vkfx.h -- C ABI of the MI355X (gfx950) batched-FFT execution library.
 *
 * This is the drop-in boundary below vkfft-rs's `NativeRuntime` HIP backend.
 * A Rust `HipNativeRuntime` binds these symbols and forwards
 * `execute_transform_f32/f64` and `submit_transform_*` to them instead of
 * lowering `TransformIr` to HIP source and JIT-compiling it with HIPRTC.
 * Citations are vkfft-rs paths (file:line) of the interface each entry
 * replaces. No HIP or torch types appear in the signatures: device buffers
 * and streams are passed as plain pointers.
 *
 * Layout conventions (vkfft-rs `Complex<T>` is #[repr(C)] {re, im},
 * src/complex.rs:4-9):
 *   - complex data is interleaved {re, im} of the plan precision;
 *   - dims are in vkfft-rs order, slowest to fastest (src/config.rs:662-666),
 *     the last dim contiguous, batches back to back;
 *   - R2C input is real (n reals per batch), output n/2+1 complex per batch;
 *     C2R is the reverse (src/program_ir.rs:6679-6711);
 *   - forward uses exp(-2 pi i jk/n); inverse exp(+2 pi i jk/n), scaled by
 *     1/n only when `normalize` is set (src/config.rs:10-15, 691).
 */
#ifndef VKFX_H
#define VKFX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. 0 = success. Negative values map onto vkfft-rs `VkFftError`
 * variants (src/error.rs:6-57); vkfx_last_error() holds the message. */
enum vkfx_status {
    VKFX_OK = 0,
    VKFX_ERR_NATIVE_UNAVAILABLE = -1,      /* NativeUnavailable{backend:"HIP"} */
    VKFX_ERR_NATIVE_RUNTIME = -2,          /* NativeRuntime{message}: a hipError_t */
    VKFX_ERR_UNSUPPORTED_KERNEL_PATH = -3, /* UnsupportedKernelPath */
    VKFX_ERR_UNSUPPORTED_PRECISION = -4,   /* UnsupportedPrecision */
    VKFX_ERR_INPUT_LENGTH_MISMATCH = -5,   /* InputLengthMismatch{expected, actual} */
    VKFX_ERR_RESOURCE_LIMIT = -6,          /* ResourceLimitExceeded */
    VKFX_ERR_INVALID_ARGUMENT = -7,        /* InvalidKernelIr / ZeroLength / invalid config */
    VKFX_ERR_ARITHMETIC_OVERFLOW = -8      /* ArithmeticOverflow */
};

/* TransformKind (src/config.rs:35-41); DCT / DST types I-IV are FFTW's
 * REDFT00/10/01/11 and RODFT00/10/01/11 (src/r2r_ir.rs:2351-2434), real in
 * and real out, both directions (inverse = the type's inverse partner, scaled
 * by 1/2(N-1), 1/2(N+1) or 1/2N when normalized; r2r_ir.rs:2318-2346). */
enum vkfx_transform {
    VKFX_C2C = 0,
    VKFX_R2C = 1,
    VKFX_C2R = 2,
    VKFX_DCT_I = 3,
    VKFX_DCT_II = 4,
    VKFX_DCT_III = 5,
    VKFX_DCT_IV = 6,
    VKFX_DST_I = 7,
    VKFX_DST_II = 8,
    VKFX_DST_III = 9,
    VKFX_DST_IV = 10
};
/* Precision (src/config.rs:108-145). The caller's buffers hold the storage
 * type; the FFT passes run on the compute type. Mixed layouts convert on the
 * device into and out of the plan's workspace. */
enum vkfx_precision {
    VKFX_F32 = 0,                     /* Precision::F32 */
    VKFX_F64 = 1,                     /* Precision::F64 */
    VKFX_F16_STORAGE_F32_COMPUTE = 2, /* Precision::F16StorageF32Compute: binary16 buffers */
    VKFX_F64_COMPUTE_F32_STORAGE = 3  /* Precision::F64ComputeF32Storage: f32 buffers */
};
enum vkfx_direction { VKFX_FORWARD = -1, VKFX_INVERSE = 1 };     /* Direction::exponent_sign */
enum vkfx_algorithm {                                            /* AxisAlgorithm, planner.rs:46-59 */
    VKFX_ALG_STOCKHAM = 0,
    VKFX_ALG_RADER = 1,
    VKFX_ALG_BLUESTEIN = 2
};

#define VKFX_MAX_RANK 4

typedef struct vkfx_context vkfx_context;
typedef struct vkfx_plan vkfx_plan;

/* DeviceProfile fields the planner and the kernels depend on
 * (src/config.rs:250-265; HIP query at src/backend/hip/runtime.rs:369-406). */
typedef struct {
    uint64_t shared_memory_bytes;      /* hipDeviceAttributeMaxSharedMemoryPerBlock */
    uint64_t shared_memory_pow2_bytes; /* largest power of two <= shared_memory_bytes */
    uint64_t max_threads_per_block;
    uint64_t warp_size;
    uint64_t compute_units;
    uint64_t global_memory_bytes;
    char name[256];
    char arch[64];
} vkfx_device_profile;

/* PlannerTuning (src/config.rs:367-380): Rader ranges and the recursive-Rader
 * opt-in. */
typedef struct {
    uint64_t min_rader_direct_prime;
    uint64_t max_rader_direct_prime; /* exclusive */
    uint64_t min_rader_fft_prime;
    uint64_t max_rader_fft_prime; /* exclusive */
    int32_t allow_recursive_fft_rader;
} vkfx_planner_tuning;

/* Plan descriptor: the part of `TransformIr` (src/application.rs:48-167) the
 * kernels need, plus the planner's per-axis decision so the library executes
 * exactly what vkfft-rs planned (src/planner.rs:168-241). With
 * use_library_planner = 1 the library fills axis_algorithm/convolution_len
 * itself from its restatement of the planner (vkfx_planner_axis). */
typedef struct {
    uint32_t rank;                          /* 1..VKFX_MAX_RANK */
    uint64_t dims[VKFX_MAX_RANK];           /* FftConfig::dimensions, slowest..fastest */
    uint64_t batch;                         /* FftConfig::batch_count (>= 1) */
    int32_t transform;                      /* vkfx_transform */
    int32_t precision;                      /* vkfx_precision */
    int32_t direction;                      /* vkfx_direction; R2C forward, C2R inverse */
    int32_t normalize;                      /* FftConfig::normalize_inverse */
    int32_t use_library_planner;            /* 1 = plan axes here */
    int32_t axis_algorithm[VKFX_MAX_RANK];  /* vkfx_algorithm per axis */
    uint64_t convolution_len[VKFX_MAX_RANK];/* Bluestein M per axis (0 = not Bluestein) */
    /* Formatted device layouts (FftConfig::with_input/output_buffer_axis_stride and
     * _batch_stride, src/config.rs:892-1002, resolved as in resolve_formatted_axis_strides,
     * config.rs:1463-1522): strides in stored elements per axis, slowest..fastest; 0 =
     * dense. The fastest axis must stay 1; each stride must cover the next faster
     * axis. For R2C the output's fastest extent is N/2+1 (C2R: the input's). */
    uint64_t in_axis_stride[VKFX_MAX_RANK];
    uint64_t out_axis_stride[VKFX_MAX_RANK];
    uint64_t in_batch_stride;               /* 0 = dense */
    uint64_t out_batch_stride;
    /* Logical zero interval [zero_left, zero_right) per axis (FftConfig::with_zero_padding,
     * config.rs:1004-1025; equal bounds = none). An element is zero when any of its
     * coordinates lies in its axis interval (zero_pad_ir.rs:607-617). Spatial domain:
     * forward input / inverse output; frequency domain (C2C only): forward output /
     * inverse input (zero_pad_ir.rs:38-46). */
    uint64_t zero_left[VKFX_MAX_RANK];
    uint64_t zero_right[VKFX_MAX_RANK];
    int32_t zero_frequency;                 /* ZeroPaddingDomain::Frequency */
    uint32_t grouped_batch[VKFX_MAX_RANK];  /* groupedBatch override (0 = automatic), a scheduling hint */
    /* Convolution, C2C only (FftConfig::with_convolution and the convolution knobs,
     * src/config.rs:595-800; ConvolutionIr / NdConvolutionIr, src/convolution_ir.rs):
     * forward FFT of every [batch][coordinate] tensor, multiply by the kernel
     * spectrum, normalized inverse FFT. The input holds batch x coordinates
     * tensors; the output holds kernel_count x coordinates tensors when
     * kernel_count > 1 (one-input fan-out, batch must be 1), else batch x
     * coordinates. kernel_spectrum: host complex values of the compute precision,
     * laid out [kernel][plane][tensor], planes = M*M (matrix), M(M+1)/2 (symmetric
     * matrix), coordinates (independent_coordinates) or 1; copied at plan time. */
    int32_t perform_convolution;
    int32_t conjugate_sequence;             /* ConvolutionConjugation::Sequence */
    int32_t cross_power_normalize;          /* cross_power_spectrum_normalization */
    uint32_t coordinate_features;           /* 0 or 1 = one coordinate */
    uint32_t matrix_convolution;            /* 0 or 1 = none; 2 or 3 = M x M matrix */
    int32_t symmetric_kernel;
    int32_t independent_coordinates;
    uint32_t kernel_count;                  /* 0 or 1 = one kernel */
    const void *kernel_spectrum;
    uint64_t kernel_spectrum_bytes;
    /* FftConfig::omit_dimension (config.rs:651, 844-853, 1053-1067): bit i set
     * leaves axis i untransformed (rank > 1; never the real axis of R2C/C2R). */
    uint32_t omit_dimension;
    /* FftConfig::with_tuning (config.rs:820-824): with custom_tuning = 0 the
     * library planner uses the AMD device tuning (PlannerTuning::for_device). */
    int32_t custom_tuning;
    vkfx_planner_tuning tuning;
} vkfx_plan_desc;

/* ---------------------------------------------------------------- context */

/* HipExecutionContext::new(device_index) (src/backend/hip/runtime.rs:1643-1656,
 * 2349-2431): selects the device, reads its profile, creates one stream of
 * default priority. Fails with VKFX_ERR_NATIVE_UNAVAILABLE without a GPU. */
int vkfx_context_create(int device_index, vkfx_context **out);
int vkfx_context_destroy(vkfx_context *ctx);

/* NativeRuntime::device_profile / device_name (src/backend/native_runtime.rs:162-166). */
int vkfx_context_profile(const vkfx_context *ctx, vkfx_device_profile *out);

/* ------------------------------------------------------------------- plan */

/* Replaces NativeSourceBackend::lower_transform + the HIPRTC compile/module
 * caches (src/backend/native.rs:696-746, src/backend/hip/runtime.rs:742-800,
 * 2109-2195): builds the kernel-launch list, uploads twiddle/chirp/spectrum
 * tables and allocates the plan's workspace once. */
int vkfx_plan_create(vkfx_context *ctx, const vkfx_plan_desc *desc, vkfx_plan **out);
/* Destroy every ticket of a plan before the plan, and every plan before the
 * context it was created on: vkfx_plan_destroy fails (VKFX_ERR_NATIVE_RUNTIME)
 * while tickets of the plan are alive, and vkfx_context_destroy fails while
 * plans or tickets of the context are alive (HipExecutionContext owns its
 * pools and streams, src/backend/hip/runtime.rs:1643-1656; tickets borrow it,
 * native_runtime.rs:406-451). */
int vkfx_plan_destroy(vkfx_plan *plan);

/* Resources of one distinct pass of a plan (NativeRuntime::
 * compiled_pass_resource_reports / theoretical_occupancy_reports,
 * src/backend/native_runtime.rs:96-131, 166-183; HIP metrics of
 * hip/runtime.rs:1849-1870): the attributes of the compiled kernel and the
 * blocks of this launch that fit on one CU. */
typedef struct {
    char pass[48];                   /* launch label (as in vkfx_plan_describe) */
    uint32_t registers_per_thread;   /* hipFuncAttributes::numRegs */
    uint32_t static_shared_bytes;    /* hipFuncAttributes::sharedSizeBytes */
    uint32_t dynamic_shared_bytes;   /* LDS the launch requests */
    uint32_t local_bytes_per_thread; /* hipFuncAttributes::localSizeBytes (scratch) */
    uint32_t max_threads_per_block;  /* hipFuncAttributes::maxThreadsPerBlock */
    uint32_t block_threads;
    uint32_t resident_blocks_per_cu; /* hipOccupancyMaxActiveBlocksPerMultiprocessor */
    uint32_t waves_per_cu;           /* resident_blocks_per_cu * ceil(block_threads / 64) */
} vkfx_pass_resources;
/* Writes up to `capacity` reports (distinct passes in launch order) and the
 * total count into *count. */
int vkfx_plan_resources(const vkfx_plan *plan, vkfx_pass_resources *out, uint32_t capacity, uint32_t *count);

/* GPU durations of a plan's FFT kernels (measurement only; no counterpart in
 * the reference, whose HIP backend publishes no timings). After
 * vkfx_plan_timing_start, every FFT kernel that vkfx_execute launches for the
 * plan, up to `max_launches` of them, is dispatched with a pair of HIP events
 * bound to that dispatch (hipExtLaunchKernel), so each pair reads the
 * kernel's own begin and end: the duration a kernel trace reports, without
 * the gaps between launches that a stream-level event pair also counts.
 * Launches past `max_launches` and non-FFT passes (boundary, copy, DCT/DST,
 * convolution multiply) run untimed. vkfx_plan_timing_stop waits for the
 * events, disarms the plan and writes one record per distinct (pass label,
 * line length, lines per launch), in launch order. Not for a plan that executes on several host threads at once. */
typedef struct {
    char pass[48];     /* launch label (as in vkfx_plan_describe) */
    uint32_t fft_len;  /* length each line of the pass transforms */
    uint32_t launches; /* timed launches with this label, length and line count */
    uint64_t lines;    /* lines of each of those launches */
    double total_ms;   /* sum of the launches' durations */
    double min_ms;
    double max_ms;
} vkfx_pass_timing;
int vkfx_plan_timing_start(vkfx_plan *plan, uint32_t max_launches);
int vkfx_plan_timing_stop(vkfx_plan *plan, vkfx_pass_timing *out, uint32_t capacity, uint32_t *count);

/* Byte sizes of one execute's input and output buffers, and of the scratch
 * a caller may pass to vkfx_execute (0 when the plan needs none). */
int vkfx_plan_io_bytes(const vkfx_plan *plan, uint64_t *in_bytes, uint64_t *out_bytes);
int vkfx_plan_workspace_bytes(const vkfx_plan *plan, uint64_t *out);

/* Output kind of a plan for the async binding. NativeProgramTicket32/64::wait
 * returns Vec<Complex32/64> for every TransformIr, and
 * finish_transform_output32/64 (src/backend/native_runtime.rs:2045-2087)
 * takes `.re` of it for C2R and DCT/DST. *real_output = 1 when the plan's
 * output holds reals (C2R, DCT/DST, real-application convolution);
 * *widened_bytes is the size of the output with every real v widened to the
 * pair {v, 0} of the storage scalar (= the output bytes for complex outputs).
 * Either pointer may be NULL. */
int vkfx_plan_output_info(const vkfx_plan *plan, int32_t *real_output, uint64_t *widened_bytes);

/* Writes a JSON description of the plan (axes, algorithms, Bluestein M,
 * four-step splits, kernel passes with grid/block/LDS) into buf. Returns the
 * number of bytes needed (excluding the NUL), or a negative status. */
int vkfx_plan_describe(const vkfx_plan *plan, char *buf, size_t cap);

/* ---------------------------------------------------------------- execute */

/* Device-resident asynchronous execute on `stream` (a hipStream_t; NULL = the
 * context's stream). Replaces HipExecutionContext::submit_prepared's kernel
 * launches (src/backend/hip/runtime.rs:1998-2107) without host copies.
 * d_in and d_out may alias for C2C (in place). d_work may be NULL, in which
 * case the plan's own workspace is used. */
int vkfx_execute(vkfx_plan *plan, const void *d_in, void *d_out, void *d_work, void *stream);

/* No counterpart in vkfft-rs: vkfx_execute for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). It runs the plan's passes with a static device
 * scratch array of the library (64 MiB, one copy per GPU, held until the
 * process ends) in place of the plan's workspace, and calls no hipMalloc,
 * hipFree or other allocating routine. Plans whose workspace exceeds 64 MiB
 * are rejected (VKFX_ERR_RESOURCE_LIMIT); plans without a workspace run as
 * with vkfx_execute. Every call on one GPU shares that GPU's array and leaves
 * its last contents there: calls that overlap on one GPU (other streams,
 * other host threads) race and must be ordered by the caller. */
int vkfx_execute_noalloc(vkfx_plan *plan, const void *d_in, void *d_out, void *stream);

/* Host round trip, the contract of NativeRuntime::execute_transform_f32/f64
 * (src/backend/native_runtime.rs:339-359): copies h_in to the device,
 * executes, copies the result to h_out and synchronises. Sizes are checked
 * against the plan (VKFX_ERR_INPUT_LENGTH_MISMATCH, native_runtime.rs:1262-1270). */
int vkfx_execute_host(vkfx_plan *plan, const void *h_in, uint64_t in_bytes, void *h_out, uint64_t out_bytes);

/* Waits for all work on the context's stream (ticket wait,
 * src/backend/hip/runtime.rs:1530-1608). */
int vkfx_context_synchronize(vkfx_context *ctx);

/* ------------------------------------------------- async tickets, chains */

typedef struct vkfx_ticket vkfx_ticket;

/* NativeAsyncRuntime::submit_transform_f32/f64_async
 * (src/backend/native_runtime.rs:406-451): copies h_in into pinned staging,
 * then queues the upload, the plan and the download on a stream of the
 * context's pool and returns at once. Each ticket owns its device buffers,
 * workspace and stream until vkfx_ticket_destroy, so several tickets (of one
 * plan or of several) may be in flight together (the reference's
 * multi-submission test, src/backend/hip/runtime.rs:3038-3095). The plan must
 * outlive its tickets; submit from one thread at a time (the context is
 * single-owner like HipExecutionContext). */
int vkfx_submit_host(vkfx_plan *plan, const void *h_in, uint64_t in_bytes, vkfx_ticket **out);

/* *ready = 1 when the ticket's work has finished, 0 otherwise; never blocks. */
int vkfx_ticket_ready(const vkfx_ticket *ticket, int32_t *ready);

/* Ticket::wait: blocks until the work is done and copies the result into
 * h_out (out_bytes must equal the plan's output bytes). The ticket stays
 * valid (wait may be repeated) until destroyed. */
int vkfx_ticket_wait(vkfx_ticket *ticket, void *h_out, uint64_t out_bytes);

/* NativeProgramTicket32/64::wait for the Rust binding
 * (src/backend/native_runtime.rs:372-401, 2045-2087): as vkfx_ticket_wait,
 * but a real-output plan's values are written as {v, 0} pairs of the storage
 * scalar, so out_bytes must equal vkfx_plan_output_info's widened_bytes. For
 * complex-output plans this is vkfx_ticket_wait. */
int vkfx_ticket_wait_complex(vkfx_ticket *ticket, void *h_out, uint64_t out_bytes);

/* Drop of a ticket (src/backend/hip/runtime.rs:1610-1619): synchronises if
 * the work is still running, then returns its buffers and stream to the
 * context's pools. */
int vkfx_ticket_destroy(vkfx_ticket *ticket);

/* HipExecutionContext::cached_transient_buffer_count / pooled_stream_count
 * (src/backend/hip/runtime.rs:1828-1840) and the in-flight submission count
 * that guards clear_runtime_caches (:2275-2284). Any pointer may be NULL. */
int vkfx_context_cache_stats(vkfx_context *ctx, uint64_t *transient_buffers, uint64_t *pooled_streams,
                             uint64_t *in_flight);
/* HipExecutionContext::clear_runtime_caches (src/backend/hip/runtime.rs:2275-2330):
 * frees the pooled transient buffers and streams of the ticket and chain
 * calls; fails (VKFX_ERR_NATIVE_RUNTIME) while tickets are in flight.
 * Plans keep their own tables and workspace until vkfx_plan_destroy. */
int vkfx_context_clear_caches(vkfx_context *ctx);

/* Device-resident chain, the HIP counterpart of
 * CudaExecutionContext::execute_program_chain_complex32
 * (src/backend/cuda/runtime.rs:1744-1809): plans[i]'s output is plans[i+1]'s
 * input and stays on the device (pooled ping-pong buffers, reused in stream
 * order). Each plan's output bytes must equal the next plan's input bytes
 * (VKFX_ERR_INPUT_LENGTH_MISMATCH otherwise). Asynchronous on `stream`
 * (NULL = the context's stream); all plans belong to one context. */
int vkfx_execute_chain(vkfx_plan *const *plans, uint32_t count, const void *d_in, void *d_out, void *stream);

/* execute_program_chain_complex32_into: host input, device-resident chain,
 * result written straight into h_out; synchronises. */
int vkfx_execute_chain_host(vkfx_plan *const *plans, uint32_t count, const void *h_in, uint64_t in_bytes,
                            void *h_out, uint64_t out_bytes);

/* Thread-local message of the last failing call on this thread. */
const char *vkfx_last_error(void);

/* Library version string. */
const char *vkfx_version(void);

/* ---------------------------------------------------- planner restatement */

/* plan_c2c_axis_algorithm_for_device for the HIP/AMD profile
 * (src/planner.rs:349-440) with PlannerTuning::for_device (src/config.rs:395-420).
 * axis_is_strided: 0 for the contiguous (last) dimension. allow_recursive_rader
 * mirrors PlannerTuning::with_recursive_fft_rader. Outputs the algorithm and,
 * for Bluestein, the convolution length M (upstream_bluestein_auto_padding,
 * src/scheduler.rs:361-373). */
int vkfx_planner_axis(uint64_t len, uint64_t batch, int32_t precision, int32_t axis_is_strided,
                      int32_t allow_recursive_rader, uint64_t shared_memory_bytes,
                      int32_t *algorithm, uint64_t *convolution_len);

/* vkfx_planner_axis with an explicit PlannerTuning (NULL: the AMD device
 * tuning), as plan_c2c_axis_algorithm_for_device with FftConfig::with_tuning. */
int vkfx_planner_axis_tuned(uint64_t len, uint64_t batch, int32_t precision, int32_t axis_is_strided,
                            const vkfx_planner_tuning *tuning, uint64_t shared_memory_bytes, int32_t *algorithm,
                            uint64_t *convolution_len);

/* upstream_bluestein_auto_padding for HIP/AMD (src/scheduler.rs:225-373). */
int vkfx_planner_bluestein_padding(uint64_t len, uint64_t batch, int32_t precision,
                                   uint64_t shared_memory_bytes, uint64_t *padded);

/* planner::next_smooth_at_least over {2,3,5,7} (src/planner.rs:684-733). */
uint64_t vkfx_planner_next_smooth(uint64_t target);

#ifdef __cplusplus
}
#endif
#endif /* VKFX_H */
