/*
 * deformops_amd: C ABI of the MI355X (gfx950) multi-scale deformable attention
 * (MSDA) library, libdeformops_amd.so.
 *
 * Every pointer is a device pointer on the current HIP device, every buffer is
 * owned by the caller (a backward workspace included), tensors are dense row-major
 * (C-contiguous), and every call is stream-ordered on `stream` (a hipStream_t; NULL
 * is the legacy default stream). The library never allocates device memory and
 * never synchronizes. A call returns
 * MSDA_OK or an error code; msda_last_error() then holds a message for the calling
 * thread.
 *
 * Shape symbols: B batch, S = sum over levels of height * width, H heads, D
 * channels per head, Q queries, L levels, P points per level.
 *
 *   value               [B, S, H, D]        value_dtype
 *   spatial_shapes      [L, 2] (height, width) per level, index_dtype
 *   level_start_index   [L]    exclusive prefix sum of height * width, index_dtype
 *   sampling_locations  [B, Q, H, L, P, 2]  loc_dtype, normalized (x, y)
 *   attention_weights   [B, Q, H, L * P]    value_dtype (raw logits when softmax != 0)
 *   output              [B, Q, H * D]       value_dtype
 *
 * Sampling follows torch.nn.functional.grid_sample(mode="bilinear",
 * padding_mode="zeros", align_corners=False): pixel = loc * size - 0.5, corners
 * outside the level contribute zero, and a sample outside -1 <= pixel < size (or
 * with a NaN coordinate) contributes nothing and has zero gradient.
 */
#ifndef DEFORMOPS_AMD_H_
#define DEFORMOPS_AMD_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MSDA_ABI_VERSION 4

/* Element types. value and attention_weights share one; locations may be
 * MSDA_F32 or the value type (MSDA_F64 only with MSDA_F64 values). */
enum msda_dtype {
  MSDA_F32 = 0,
  MSDA_F16 = 1,
  MSDA_BF16 = 2,
  MSDA_F64 = 3,
};

/* Element types of spatial_shapes and level_start_index. */
enum msda_index_dtype {
  MSDA_I64 = 0,
  MSDA_I32 = 1,
};

/* Bits of the flags argument. */
enum msda_flags {
  MSDA_SOFTMAX = 1,               /* normalize attention_weights over the L * P points */
  MSDA_ACCUMULATE_GRAD_VALUE = 2, /* backward: add into grad_value instead of overwriting it */
  MSDA_GRAD_VALUE_ATOMIC = 4,     /* backward: grad_value by global atomics (see msda_backward) */
};

/* Kernel paths msda_set_path_override can force. */
enum msda_path_bits {
  MSDA_PATH_NO_MFMA = 1,     /* grad_value on the VALU owner kernel instead of the matrix cores */
  MSDA_PATH_ATOMIC_SORT = 2, /* bucket sort publishing counts with global atomics */
  MSDA_PATH_TILE8 = 4,       /* matrix-core grad_value on 8 x 8 tiles at every level */
};

/* Return codes. */
enum msda_status {
  MSDA_OK = 0,
  MSDA_ERR_INVALID = 1,     /* a null pointer, a negative size or an unknown dtype */
  MSDA_ERR_UNSUPPORTED = 2, /* a valid call this build has no kernel for */
  MSDA_ERR_HIP = 3,         /* a HIP runtime error at launch */
};

/*
 * Forward: output[b, q, h*D + d] = sum over (l, p) of
 *   w[b,q,h,l,p] * bilinear(value[b, level l, :, h, d], loc[b,q,h,l,p]),
 * with w = attention_weights, or their softmax over the L * P points of each
 * (b, q, h) when flags has MSDA_SOFTMAX. The output is written in full (zeros when
 * L * P == 0).
 *
 * Replaces the forward operator the reference binds through the torch
 * dispatcher: deformops_cuda::msda_fp32acc[_softmax]_forward
 * (sources/deformops/backends/cuda/_schema.py:18-23, boxed entry
 * include/msda_boxed.cuh:14-28, host launch include/msda_launch.cuh:63-138).
 */
int msda_forward(const void* value, int value_dtype,
                 const void* spatial_shapes, const void* level_start_index,
                 int index_dtype,
                 const void* sampling_locations, int loc_dtype,
                 const void* attention_weights,
                 void* output,
                 int64_t batch, int64_t spatial, int64_t heads, int64_t channels,
                 int64_t queries, int64_t levels, int64_t points,
                 int flags, void* stream);

/*
 * Backward of msda_forward for the upstream gradient grad_output [B, Q, H * D]
 * (value_dtype). Writes
 *   grad_value               [B, S, H, D]        value_dtype
 *   grad_sampling_locations  [B, Q, H, L, P, 2]  loc_dtype
 *   grad_attention_weights   [B, Q, H, L * P]    value_dtype (w.r.t. the logits
 *                                                 under MSDA_SOFTMAX)
 * Every element of grad_value gets its gradient from one owner, which sums all its
 * contributions in fp32 (fp64 for MSDA_F64) and stores once; with
 * MSDA_ACCUMULATE_GRAD_VALUE the previous contents are added to that sum. No
 * atomics touch grad_value, it needs no zero-fill, and there is no float32 copy.
 * For bf16, f16 and float values the owner sums on the matrix cores with each
 * weight * grad_out product formed from 16-bit parts (relative error at most 2^-16
 * for bf16, 2^-22 for f16 while the weight's low part is a normal f16 number, and
 * 3 * 2^-16 for float; see msda.hip).
 * The order in which an element's contributions are summed follows the order the
 * bucket sort gives the samples, which depends on the order of its LDS atomics
 * across waves; so the last bits of grad_value may vary between runs. The other two
 * gradients are written in full, zeros included.
 *
 * With MSDA_GRAD_VALUE_ATOMIC, or when two valid levels of the table share
 * positions of S (found on the device), grad_value is instead zero-filled (unless
 * MSDA_ACCUMULATE_GRAD_VALUE) and every sample adds weight * grad_out into its
 * corners with global atomics in the value dtype (fp32 / fp64 adds, packed bf16 /
 * f16 pair adds), the mechanism of the reference's kernels
 * (include/interpolate.cuh:146-175, and the native-dtype atomics of the Triton
 * zero-buffer backward, backends/triton/_kernels/msda_query_tiled.py:435-483).
 * Overlapping levels then sum their contributions into a shared element, as the
 * reference's eager and atomic paths do. A 16-bit grad_value accumulates in its own
 * dtype there, so it carries one rounding per contribution. While the call
 * runs, its outputs serve as its scratch (a bucket sort of the samples by pyramid
 * tile): grad_sampling_locations holds the sorted sample indices,
 * grad_attention_weights the bucket counters, and grad_value the samples' keys
 * until the owners overwrite it (with MSDA_ACCUMULATE_GRAD_VALUE the keys are
 * recomputed instead, and grad_value holds only its previous contents);
 * all three hold their gradients when the call completes. So the call needs no
 * memory beyond its outputs, and the three gradient buffers must not alias each
 * other or the inputs. grad_sampling_locations must be 4-byte aligned.
 *
 * Replaces deformops_cuda::msda_fp32acc[_softmax]_backward
 * (sources/deformops/backends/cuda/_schema.py:24-29, include/msda_boxed.cuh:32-53,
 * include/msda_launch.cuh:140-275), which needs float32 copies of every input and
 * a float32 scratch grad_value for 16-bit inputs.
 */
int msda_backward(const void* value, int value_dtype,
                  const void* spatial_shapes, const void* level_start_index,
                  int index_dtype,
                  const void* sampling_locations, int loc_dtype,
                  const void* attention_weights,
                  const void* grad_output,
                  void* grad_value, void* grad_sampling_locations,
                  void* grad_attention_weights,
                  int64_t batch, int64_t spatial, int64_t heads, int64_t channels,
                  int64_t queries, int64_t levels, int64_t points,
                  int flags, void* stream);

/*
 * msda_backward with a caller workspace of at least msda_backward_workspace_size
 * bytes for the same sizes (device memory, 256-byte aligned; its contents are
 * ignored and left undefined). Writes the same three gradients. The bucket sort keeps
 * its counters and sorted sample indices in the workspace instead of
 * grad_attention_weights and grad_sampling_locations, so the location and weight
 * gradient kernel no longer has to run after it: where that kernel adds nothing into
 * grad_value (the matrix-core owners take every level, overlapping ones included,
 * and MSDA_GRAD_VALUE_ATOMIC is off) and the call has at least 2^21 samples, the call
 * forks it onto a side stream of the calling thread (created on the first such call
 * per thread and device, default priority) beside the sort and the grad_value
 * kernel, and joins the caller's stream at the end of the call (with MSDA_SOFTMAX,
 * before the grad_value kernel, which then reads the softmax statistics grad_sample
 * leaves): 9-13 us less GPU time at B = 4, Q = 21,504 in bf16, 21 us with softmax.
 * The fork and join cost the calling thread about 45 us, so smaller calls, whose
 * GPU time would not hide that, keep one stream.
 * Work before the call on `stream` happens before all of it, and work after the call
 * after all of it, so it stays stream-ordered and can be captured in a HIP graph.
 * The workspace holds 4 bytes per sample, then at least as many bytes as
 * grad_attention_weights, and room for the bucket counters of the largest tile count
 * the sizes allow, so that the grad_value kernel never needs its fallback launch
 * (49.5 MB at B = 4, Q = 21,504, H = 8, L = 3, P = 4 in bf16; 5.2 MB for 300 queries
 * on a 17,821-position pyramid in float32). With MSDA_SOFTMAX it also holds one
 * softmax statistic per (b, q, h) (4 bytes, 8 in float64: 2.75 MB more at that
 * workload), which the forked grad_sample writes, so that no statistics pass follows
 * the sort. A smaller workspace that still holds the indices and
 * grad_attention_weights' bytes works too, with that fallback and that pass where
 * they are needed; a null or yet smaller one makes the call msda_backward.
 *
 * Replaces the same backward operator as msda_backward.
 */
int msda_backward_workspace(const void* value, int value_dtype,
                            const void* spatial_shapes, const void* level_start_index,
                            int index_dtype,
                            const void* sampling_locations, int loc_dtype,
                            const void* attention_weights,
                            const void* grad_output,
                            void* grad_value, void* grad_sampling_locations,
                            void* grad_attention_weights,
                            int64_t batch, int64_t spatial, int64_t heads, int64_t channels,
                            int64_t queries, int64_t levels, int64_t points,
                            int flags, void* workspace, int64_t workspace_bytes, void* stream);

/* Bytes of workspace msda_backward_workspace takes for these sizes and flags (only
 * MSDA_SOFTMAX changes it). Host only. No counterpart in the reference (its scratch
 * is allocated inside the op). */
int msda_backward_workspace_size(int value_dtype, int64_t batch, int64_t spatial, int64_t heads,
                                 int64_t channels, int64_t queries, int64_t levels, int64_t points,
                                 int flags, int64_t* bytes);

/*
 * msda_backward_workspace with the workspace in a static device array of 64 MiB
 * (`scratch` in msda.hip, one per device, held from the module's load on that device
 * until the process ends): a backward that allocates nothing, for callers that cannot
 * call hipMalloc (code under HIP graph capture, tight serving loops, harnesses that
 * forbid allocation). No counterpart in the reference. Same arguments and results as
 * msda_backward, kernels in turn on `stream` (no side stream). Sizes whose workspace
 * exceeds 64 MiB (msda_backward_workspace_size; more than 2^23 samples in 4-byte
 * dtypes) fail with MSDA_ERR_INVALID before any launch. Every call on a device shares
 * that device's array, so calls that overlap on one device (two streams, two threads)
 * race and give wrong gradients: serialize them.
 */
int msda_backward_no_alloc(const void* value, int value_dtype,
                           const void* spatial_shapes, const void* level_start_index,
                           int index_dtype,
                           const void* sampling_locations, int loc_dtype,
                           const void* attention_weights,
                           const void* grad_output,
                           void* grad_value, void* grad_sampling_locations,
                           void* grad_attention_weights,
                           int64_t batch, int64_t spatial, int64_t heads, int64_t channels,
                           int64_t queries, int64_t levels, int64_t points,
                           int flags, void* stream);

/* The message of the calling thread's last failed call ("" if none). Replaces the
 * std::runtime_error text of TORCH_CHECK (include/stable_compat.cuh:33-46). */
const char* msda_last_error(void);

/* MSDA_ABI_VERSION of the loaded library. */
int msda_abi_version(void);

/* Forces kernel paths of later calls in this process (msda_path_bits; 0 restores
 * the library's own choice) and returns the previous bits. No counterpart in the
 * reference: it lets a test run every grad_value and sort path the library has on
 * inputs where another path would be chosen. Results are the same on every path
 * up to rounding. Not meant to be changed while calls run on other threads. */
int msda_set_path_override(int paths);

/* Makes later backward calls (any of the three entry points) on the calling thread
 * record the four HIP events events[0..3] (hipEvent_t, created by the caller) on
 * their stream: before the bucket sort, after the sort (and the softmax
 * statistics), after grad_value, and after grad_sample; count 0 stops it. While the
 * events are set the kernels run in that order on the caller's stream (no side
 * stream). No counterpart in the reference: a measurement hook, so that a benchmark
 * can time each phase of a backward call (bench.py rates each kernel by its L2
 * requests per second). */
int msda_set_phase_events(void* const* events, int count);

/* The launch layout msda_forward / msda_backward would use for these sizes:
 * channels per lane, lanes per (query, head) unit and waves per workgroup. Host
 * only; lets a caller or a test check the geometry without a GPU. Returns MSDA_OK
 * or the error code the compute call would return. */
int msda_launch_geometry(int value_dtype, int64_t batch, int64_t spatial,
                         int64_t heads, int64_t channels, int64_t queries,
                         int64_t levels, int64_t points, int backward,
                         int* channels_per_lane, int* lanes_per_unit,
                         int* waves_per_block, int64_t* num_blocks);

#ifdef __cplusplus
}
#endif

#endif /* DEFORMOPS_AMD_H_ */
