/*
 * gdn_prefill.h - C ABI of the MI355X (gfx950) Gated Delta Net prefill.
 *
 * Variable-length prefill over N sequences packed along the token axis, in
 * the reference's tensor layouts (solution/triton/prefill_kernel.py:96-114):
 *
 *   q, k        [L, H,  K]        bf16   (K = 128, H <= 32767; L = total tokens)
 *   v           [L, HV, V]        bf16   (V = 128, HV % H == 0)
 *   state       [N, HV, V, K]     fp32   k-last; NULL means zeros
 *   A_log       [HV]              fp32
 *   a, b        [L, HV]           bf16
 *   dt_bias     [HV]              fp32
 *   cu_seqlens  [N + 1]           int32  sequence s is tokens
 *                                        [cu_seqlens[s], cu_seqlens[s+1])
 *   output      [L, HV, V]        bf16
 *   new_state   [N, HV, V, K]     fp32   may be the same buffer as state
 *
 * For each sequence and v-head hv (q/k head hv / (HV/H)), token after token,
 * the decode step of gdn_decode.h against the running state; the state
 * after the sequence's last token goes to new_state (zeros for a sequence
 * with no tokens, as the reference).  Evaluated chunkwise (64 tokens) with
 * MFMA; arithmetic in fp32 except the bf16 x bf16 products of the inputs
 * themselves (K K^T, Q K^T), which are exact in fp32 accumulation.
 *
 * cu_seqlens is read on the device.  It should be non-decreasing with
 * cu_seqlens[0] = 0 and cu_seqlens[N] = L, as the reference requires; token
 * ranges are clamped to [0, L] on the device, so other contents give
 * unspecified results but no out-of-bounds access.
 *
 * All pointers are device pointers.  The call is asynchronous on
 * `hip_stream`, allocates nothing, and returns 0 or a nonzero hipError_t
 * (hipErrorInvalidValue = 1 for bad sizes, null or misaligned pointers, a
 * short workspace, or a new_state that partly overlaps state).
 */
#ifndef GDN_PREFILL_H
#define GDN_PREFILL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Bytes of device workspace gdn_prefill needs for L total tokens, N
 * sequences, H q/k heads and HV v-heads: per-chunk intermediates (14 KiB
 * per chunk per v-head, for min(ceil(L / 64) + N, L) chunks, the most a
 * well-formed batch has, rounded up to 256 bytes), a 16-byte table entry per
 * chunk and 4 bytes per sequence, each part rounded up to 256 bytes; for a
 * batch scanned in segments (at most 64 sequences, N x HV <= 256, sequences
 * of the mean length long enough that segments of 2 or more chunks, the
 * length minimising the estimated critical path of the two segment scans
 * and the combine, beat the plain scan), also 3 x 64 KiB per segment per
 * v-head: one sequence's ceil(ceil(L / 64) / len) segments, several
 * sequences' (min(ceil(L / 64) + N, L) + N (len - 1)) / len.
 * 0 for invalid sizes.
 * The reference's FLA path allocates its intermediates per call inside
 * chunk_gated_delta_rule (solution/triton/fla_prefill_code.py:1726-1776);
 * here the caller provides them.
 */
size_t gdn_prefill_workspace_bytes(int total_seq_len, int num_seqs, int H, int HV);

/*
 * One prefill over all sequences.  Replaces the reference's prefill entry
 * points, which take the same tensors, cu_seqlens and scale:
 *   solution/triton/prefill_kernel.py:10-58   kernel_prefill_fla_chunk (DPS)
 *   solution/triton/prefill_kernel.py:85-183  kernel_prefill_reference
 * Differences: sizes are explicit, K and V must be 128, the q/k L2-norm is an
 * explicit flag (off in the reference's prefill, prefill_kernel.py:45), the
 * workspace (256-byte aligned, gdn_prefill_workspace_bytes long) comes from
 * the caller, `scale` is already resolved (None/0 -> 1/sqrt(K) in the
 * Python caller), and bad arguments return an error instead of launching.
 * q, k, v, output, state and new_state must be 16-byte aligned.
 * Launches one kernel when total_seq_len <= gdn_prefill_token_path_max_tokens()
 * (and num_seqs <= 65535): the token-by-token kernel; one kernel when
 * total_seq_len is past that but at most 64 (every sequence one chunk) and
 * num_seqs x HV <= 128: the one-chunk kernel, each workgroup of which
 * prepares its sequence's chunk in LDS and scans it; else the chunkwise
 * kernels: the chunk-offsets
 * scan (not for one sequence, nor for at most 64 whose slots the kernels
 * find themselves), preparation, scan (for a few sequences whose scans would
 * leave most CUs idle: their segments scanned at once in two launches with
 * the combination of their starts between them).  For 2..64 sequences of at
 * most gdn_prefill_token_path_max_tokens() tokens on average, the
 * token-by-token kernel is launched first: it runs only if every sequence
 * is that short (read from cu_seqlens on the device), and the chunkwise
 * kernels after it then return at once; otherwise they run the whole batch.
 * gdn_prefill_dispatches gives the launch count.
 */
int gdn_prefill(const void* q, const void* k, const void* v, const float* state,
                const float* A_log, const void* a, const float* dt_bias, const void* b,
                const int32_t* cu_seqlens, float scale, void* output, float* new_state,
                int total_seq_len, int num_seqs, int H, int HV, int K, int V,
                int use_qk_l2norm, void* workspace, size_t workspace_size,
                void* hip_stream);

/*
 * Measurement hook, no counterpart in the reference: gdn_prefill with
 * events[0..3] (hipEvent_t, all non-null) recorded on hip_stream before the
 * offsets, preparation and scan launches and after the scan, so that
 * hipEventElapsedTime gives each kernel's time (the segmented scan's two or
 * three launches lie between events 2 and 3).  Without an offsets launch
 * (one sequence, or few: see gdn_prefill_dispatches) events 0 and 1 are
 * recorded back to back; with one kernel (the token-by-token kernel or the
 * one-chunk kernel) events 0..2 are, and its launch lies between events 2
 * and 3.  Nothing is recorded when num_seqs is 0.
 */
int gdn_prefill_timed(const void* q, const void* k, const void* v, const float* state,
                      const float* A_log, const void* a, const float* dt_bias, const void* b,
                      const int32_t* cu_seqlens, float scale, void* output, float* new_state,
                      int total_seq_len, int num_seqs, int H, int HV, int K, int V,
                      int use_qk_l2norm, void* workspace, size_t workspace_size,
                      void* hip_stream, void* const* events);

/* Bytes of the fixed per-GPU workspace gdn_prefill_noalloc uses: 128 MiB. */
#define GDN_PREFILL_NOALLOC_SCRATCH_BYTES ((size_t)128 << 20)

/*
 * gdn_prefill without a caller-provided workspace and without allocating:
 * the workspace is a fixed device array of GDN_PREFILL_NOALLOC_SCRATCH_BYTES
 * in this library, one per GPU, held from the library's first use on that
 * GPU until the process ends.  No counterpart in the reference (whose FLA
 * path allocates its intermediates per call, fla_prefill_code.py:1726-1776):
 * for callers that cannot allocate device memory -- code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation.
 * Sizes whose workspace (gdn_prefill_workspace_bytes) exceeds the array
 * return hipErrorOutOfMemory (2) before anything is launched; other
 * arguments and results as gdn_prefill, on the current device's array.
 * Every call on one GPU shares that array, and nothing in it needs to start
 * at zero: calls on one stream run one after another, but calls that overlap
 * on one GPU (different streams, or different host threads without
 * ordering) race on it and give wrong results.
 */
int gdn_prefill_noalloc(const void* q, const void* k, const void* v, const float* state,
                        const float* A_log, const void* a, const float* dt_bias, const void* b,
                        const int32_t* cu_seqlens, float scale, void* output, float* new_state,
                        int total_seq_len, int num_seqs, int H, int HV, int K, int V,
                        int use_qk_l2norm, void* hip_stream);

/*
 * Total tokens up to which gdn_prefill runs the token-by-token path: one
 * launch in which each workgroup applies the recurrence to its sequence's
 * tokens with its slice of the state in registers (no sequence is longer
 * than the total).  No counterpart in the reference; for callers that count
 * dispatches or time the two paths.
 */
int gdn_prefill_token_path_max_tokens(void);

/*
 * Kernel launches gdn_prefill makes for these sizes: 0 for no sequences, 1
 * for the token-by-token kernel or the one-chunk kernel; else the chunkwise
 * kernels -- 2 (preparation,
 * scan), or 4 for a batch scanned in segments (preparation, first segment
 * scan, combine, second segment scan) -- plus 1 for the chunk-offsets scan
 * first, except for a single sequence and for at most 64 with at most 2048
 * (slot, v-head) pairs (min(ceil(L / 64) + N, L) x HV; the kernels then find
 * the chunk slots from cu_seqlens themselves), plus 1 for the token-by-token
 * kernel launched before them for 2..64 sequences of at most
 * gdn_prefill_token_path_max_tokens() tokens on average.  No counterpart in
 * the reference; for callers that attribute kernel traces to calls.
 */
int gdn_prefill_dispatches(int total_seq_len, int num_seqs, int HV);

/* ABI version of this header: 6 (5 had no gdn_prefill_noalloc; 4 had no
 * gdn_prefill_dispatches; 3 had no gdn_prefill_token_path_max_tokens; 2 had
 * no gdn_prefill_timed; 1 had no H in gdn_prefill_workspace_bytes). */
int gdn_prefill_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* GDN_PREFILL_H */
