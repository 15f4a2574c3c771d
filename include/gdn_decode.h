/*
 * gdn_decode.h - C ABI of the MI355X (gfx950) Gated Delta Net decode step.
 *
 * Decode steps of the gated delta rule over a batch of recurrent states, in
 * the reference's tensor layouts (T = 1 token per sequence for the
 * reference's decode; T > 1 for multi-token decode):
 *
 *   q, k       [B, T, H,  K]   bf16   (K = 128, H <= 32767)
 *   v          [B, T, HV, V]   bf16   (V = 128, HV % H == 0, GVA ratio HV/H)
 *   state      [B, HV, V, K]   fp32   "k-last": element (k, v) at v*K + k
 *                                     (bf16 with gdn_decode_steps' state_bf16);
 *                                     NULL starts every sequence from zeros
 *   A_log      [HV]            fp32
 *   a, b       [B, T, HV]      bf16   ([B, HV] is the same memory at T = 1)
 *   dt_bias    [HV]            fp32
 *   output     [B, T, HV, V]   bf16
 *   new_state  [B, HV, V, K]   as state; may be the same buffer as state
 *
 * Per (batch b, v-head hv), with h = hv / (HV / H), for t = 0 .. T-1:
 *   g     = exp(-exp(A_log[hv]) * softplus(a[b,t,hv] + dt_bias[hv]))
 *   beta  = sigmoid(b[b,t,hv])
 *   q, k  = l2norm(q[b,t,h]), l2norm(k[b,t,h])  only when use_qk_l2norm != 0
 *   S     = g * S                                (S = state[b,hv] at t = 0)
 *   S    += k (x) beta * (v[b,t,hv] - S k)       rank-1 delta-rule update
 *   output[b,t,hv] = bf16(scale * S q)
 * and new_state[b,hv] = S after the last token.  Arithmetic is fp32; a bf16
 * state is widened on load and rounded to nearest even on store.
 *
 * All pointers are device pointers, dense and row-major in the shapes above.
 * Every entry point is asynchronous on `hip_stream` (a hipStream_t, NULL for
 * the null stream), allocates nothing, and returns 0 on success or a nonzero
 * hipError_t code.  Arguments are validated on the host before any launch
 * (hipErrorInvalidValue = 1 for bad sizes, null or misaligned pointers;
 * state, new_state, q, k, v and output must be 16-byte aligned).
 */
#ifndef GDN_DECODE_H
#define GDN_DECODE_H

#ifdef __cplusplus
extern "C" {
#endif

/*
 * One decode step with the library's launch-shape choice for (B, HV).
 *
 * Replaces the reference's native decode entry points, which take the same
 * eleven tensors plus `scale` and launch the fused decode kernel on the
 * caller's current stream:
 *   solution/cuda/kernel.cu:405-443  KernelCudaV4 / kernel_cuda_v4 (TVM FFI)
 *   solution/cuda/kernel.cu:216-254  KernelCuda   / kernel_cuda    (TVM FFI)
 *   solution/triton/kernel.py:150-197 kernel_fla_recurrent (Triton launch)
 * Differences: sizes are explicit integers instead of DLPack views, K and V
 * must be 128 (the reference hard-codes BK = 128, kernel.cu:24), the q/k
 * L2-norm is an explicit flag (off in every reference decode entry,
 * kernel.py:146), and bad arguments return an error instead of launching.
 * `scale` must already be resolved (the reference's None/0 -> 1/sqrt(K)
 * default, kernel.py:163-164, is applied by the Python caller).
 */
int gdn_decode_step(const void* q, const void* k, const void* v,
                    const float* state, const float* A_log, const void* a,
                    const float* dt_bias, const void* b, float scale,
                    void* output, float* new_state,
                    int B, int H, int HV, int K, int V,
                    int use_qk_l2norm, void* hip_stream);

/*
 * T >= 1 tokens per sequence, with an fp32 (state_bf16 = 0) or bf16
 * (state_bf16 = 1) state; otherwise as gdn_decode_step, which is this call
 * with T = 1 and an fp32 state.  The state is read once and written once
 * whatever T is.
 * Counterpart of FlashInfer's gated_delta_rule_decode_pretranspose, which
 * the reference calls for its fi-baseline entry
 * (solution/triton/kernel.py:135-147) and whose T = 1..4 and bf16-state
 * support the reference records (findings/fi-gdn-decode-kernel.md:11-16).
 */
int gdn_decode_steps(const void* q, const void* k, const void* v,
                     const void* state, const float* A_log, const void* a,
                     const float* dt_bias, const void* b, float scale,
                     void* output, void* new_state,
                     int B, int T, int H, int HV, int K, int V,
                     int state_bf16, int use_qk_l2norm, void* hip_stream);

/*
 * gdn_decode_steps with an explicit launch shape: each wavefront owns
 * 4 * rows_per_lane_group consecutive-row groups of state rows (16 lanes per
 * row), each workgroup holds `waves_per_block` wavefronts, and a (b, hv) head
 * is split over 128 / (4 * rows_per_lane_group * waves_per_block) workgroups.
 * rows_per_lane_group and waves_per_block are each one of 1, 2, 4, 8 and
 * their product is at most 32.  cache_policy selects how the state stream
 * is accessed: 0 ordinary loads and stores, 1 nontemporal loads and stores,
 * 2 nontemporal stores only, 3 nontemporal loads only.  With T > 1, a
 * bf16 state or a NULL state, cache_policy is 0 or 1.
 * rows_per_lane_group 16, 32 or 64 (T = 2..4 only, cache_policy 1) selects
 * the block kernel instead: the T tokens' dot products are taken against the
 * starting state on the matrix cores and the state is updated once; each
 * wavefront owns rows_per_lane_group consecutive state rows as 16-row MFMA
 * tiles, rows_per_lane_group * waves_per_block <= 128, and a head is split
 * over 128 / (rows_per_lane_group * waves_per_block) workgroups.
 * start_event / stop_event (hipEvent_t, may be
 * NULL) are stamped with the kernel's own start and end timestamps
 * (hipExtLaunchKernelGGL), so hipEventElapsedTime gives the kernel duration
 * without event-marker overhead.  Used for launch-shape sweeps and timing.
 * Counterpart of the reference's fixed launch choice (BV = 8 rows and
 * num_warps = 8 if B <= 4 else 4, solution/triton/kernel.py:168-197; grid
 * (V/8, B*HV), solution/cuda/kernel.cu:229-235,418-424).
 */
int gdn_decode_step_shaped(const void* q, const void* k, const void* v,
                           const void* state, const float* A_log,
                           const void* a, const float* dt_bias, const void* b,
                           float scale, void* output, void* new_state,
                           int B, int T, int H, int HV, int K, int V,
                           int state_bf16, int use_qk_l2norm,
                           int rows_per_lane_group,
                           int waves_per_block, int cache_policy,
                           void* start_event, void* stop_event,
                           void* hip_stream);

/*
 * Measurement instrument, no counterpart in the reference: one T = 1 step
 * (fp32 state, not NULL; B <= 65535) through an instrumented copy of the
 * single-token kernel with the given launch shape (rows_per_lane_group x
 * waves_per_block one of 1x1, 2x2, 4x1, 8x1, 2x4; nontemporal state
 * access) that also writes 8 clock stamps per wavefront to `stamps`
 * (stamp_capacity entries, at least 8 per wavefront: the launch has
 * B x HV x 128 / (4 x rows_per_lane_group) wavefronts; wavefront w of
 * linear block i at entry 8 * (i * waves_per_block + w)): the real-time
 * clock (100 MHz) at entry; the shader clock at entry, after the state
 * loads are issued, after the per-head math (the small inputs arrived),
 * when the state has arrived, after the state stores are issued, and when
 * every store has completed; the real-time clock at the end.  The phases
 * of the reference's clock64 instrumentation plan
 * (findings/potential-cuda-improvement.md:457-496) on this kernel.
 */
int gdn_decode_step_stamped(const void* q, const void* k, const void* v, const float* state,
                            const float* A_log, const void* a, const float* dt_bias,
                            const void* b, float scale, void* output, float* new_state,
                            int B, int H, int HV, int K, int V, int use_qk_l2norm,
                            int rows_per_lane_group, int waves_per_block,
                            unsigned long long* stamps, long long stamp_capacity,
                            void* hip_stream);

/*
 * Launch shape gdn_decode_steps would use for B sequences of T tokens over
 * HV v-heads with an fp32 (state_bf16 = 0) or bf16 (1) state: writes
 * rows_per_lane_group, waves_per_block, cache_policy and the workgroup
 * count.  Returns 0, or hipErrorInvalidValue for B < 0, T < 1, HV <= 0, a
 * state_bf16 other than 0 or 1, or null outputs.
 * No reference counterpart (the reference's choice is inline in its
 * wrappers, solution/triton/kernel.py:168-174).
 */
int gdn_decode_launch_shape(int B, int T, int HV, int state_bf16,
                            int* rows_per_lane_group, int* waves_per_block,
                            int* cache_policy, long long* num_blocks);

/*
 * A decode call bound once: gdn_decode_plan_create validates the arguments
 * of gdn_decode_steps (the same pointers, sizes and flags) and resolves the
 * launch shape, so that running it again is one launch per plan with no
 * per-call checks.  The pointed-to buffers must stay allocated while the
 * plan (or a graph built from it) is used; their contents may change
 * between runs (the caller writes the next token's q, k, v, a and b into
 * them).  A plan records the device current at its creation (the
 * buffers' device); gdn_decode_plan_run launches plans[0 .. n-1] in order on
 * hip_stream (a stream of their device), each with its plan's device made
 * current for the launch and the caller's restored after.
 * gdn_decode_plan_create returns the codes gdn_decode_steps
 * returns for the same arguments (hipErrorOutOfMemory if the host
 * allocation fails) and sets *plan to NULL on error.
 *
 * The reference's B = 1 serving notes plan exactly this for its decode step
 * (launch overhead dominating a ~3 us kernel, findings/potential-cuda-
 * improvement.md:143-147,539): its entries validate and look up the stream
 * on every call (solution/cuda/kernel.cu:405-443).
 */
typedef struct gdn_decode_plan gdn_decode_plan;

int gdn_decode_plan_create(const void* q, const void* k, const void* v, const void* state,
                           const float* A_log, const void* a, const float* dt_bias,
                           const void* b, float scale, void* output, void* new_state,
                           int B, int T, int H, int HV, int K, int V, int state_bf16,
                           int use_qk_l2norm, gdn_decode_plan** plan);
int gdn_decode_plan_run(const gdn_decode_plan* const* plans, int n, void* hip_stream);
void gdn_decode_plan_destroy(gdn_decode_plan* plan);

/*
 * One HIP graph of the launches of plans[0 .. n-1] (n >= 1), in order,
 * recorded by stream capture on a private stream of the current device and
 * instantiated once; gdn_decode_graph_launch replays it on hip_stream (a
 * stream of the same device), as one submission for all n steps (e.g. the
 * GDN layers of a model's decode step).  The plans may be destroyed after
 * gdn_decode_graph_create; their buffers may not.  The graph holds no
 * memset nodes.  Counterpart of the CUDA-graph capture the reference's
 * serving notes plan (findings/potential-cuda-improvement.md:143-147).
 */
typedef struct gdn_decode_graph gdn_decode_graph;

int gdn_decode_graph_create(const gdn_decode_plan* const* plans, int n,
                            gdn_decode_graph** graph);
int gdn_decode_graph_launch(const gdn_decode_graph* graph, void* hip_stream);
void gdn_decode_graph_destroy(gdn_decode_graph* graph);

/*
 * Human-readable text for a return code of the functions above
 * (hipGetErrorString).  The reference has no error path
 * (solution/cuda/kernel.cu:216-252 never checks a launch).
 */
const char* gdn_decode_error_string(int code);

/* ABI version of this header: 6 (5 had no block kernel shapes; 4 had no
 * gdn_decode_step_stamped; 3 had no plans or graphs and no NULL state). */
int gdn_decode_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* GDN_DECODE_H */
