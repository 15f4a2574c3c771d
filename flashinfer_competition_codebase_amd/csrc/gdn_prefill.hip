// gdn_prefill.hip - Gated Delta Net prefill (variable-length sequences) for
// gfx950 (MI355X), chunkwise with MFMA.
//
// Semantics: the reference's prefill (solution/triton/prefill_kernel.py:
// 85-183) -- per sequence of cu_seqlens, the decode step applied token after
// token to the running fp32 state (k-last [HV, V, K] per sequence), output
// per token, the final state per sequence.  The recurrence is evaluated in
// chunks of C = 64 tokens (the chunkwise form of the gated delta rule): with
// gamma_i the cumulative log-decay inside a chunk and S_0 the state ([K, V])
// at its start,
//   A     = strict_lower(beta_i e^(gamma_i - gamma_j) k_i . k_j)
//   T     = (I + A)^-1                                 (unit lower triangular)
//   X     = V - diag(e^gamma) K S_0        (what the decayed state misses)
//   Delta = T diag(beta) X                 (the per-token delta-rule corrections;
//                                           = U - W S_0 of the WY form)
//   O     = scale [diag(e^gamma) Q S_0 + (Q K^T (.) M) Delta],
//           M_ij = e^(gamma_i - gamma_j) for j <= i
//   S_C   = e^(gamma_C) S_0 + (diag(e^(gamma_C - gamma)) K)^T Delta
// Every exponent is <= 0.  With the q/k L2-norm on, the row norms enter as
// per-row scale factors of the same products.
//
// Prefills of at most kSmallTokens (56) tokens in all (so every sequence is
// that short) skip the chunkwise machinery: one launch of the decode kernel's
// variable-length mode (gdn_decode_kernel.h) applies the recurrence token by
// token with the state in registers, one workgroup per (sequence, v-head,
// row tile), reading each sequence's token range from cu_seqlens on the
// device.  Prefills of 57 to 64 tokens in all (every sequence one chunk)
// whose (sequence, v-head) pairs fill at most half the CUs run one launch of
// the one-chunk kernel: each half-state scan workgroup prepares its
// sequence's chunk in its own LDS (kernel 2's code) and scans it (kernel
// 3's), so the slot never goes through the workspace.  Larger prefills run
// the chunkwise kernels -- after the token kernel's launch, for 2..64
// sequences that may all be at most 56 tokens long (the host knows only the
// total): it runs only if every sequence is, and the chunkwise kernels then
// return at once.
//
// Kernels (one stream, in order):
//   1. chunk_offsets: one workgroup turns cu_seqlens into the first chunk
//      slot of every sequence (token ranges clamped to [0, L]) by a scan,
//      and writes each slot's sequence, first token and token count.  With
//      one sequence, or a few (their slots found in the kernels), it is not
//      launched.
//   2. prep, grid (chunk slots, H) -- or (chunk slots, HV), one v-head a
//      workgroup, when all of those fit on the GPU at once -- four
//      workgroups per CU: what does not depend on the state, for all chunks
//      at once -- K K^T (bf16 MFMA: the inputs are bf16, once per q/k head
//      and workgroup), then per v-head the gates and
//      gamma and T by block recursion (fp32 MFMA) -- into a 14 KiB workspace
//      slot per (chunk, v-head): the lower blocks of T diag(beta), split
//      into bf16 hi + lo in the order the scan's MFMAs read them, and the
//      row scales.
//   3. scan, one workgroup per (sequence, v-head), XCD-aware order: the
//      sequential part chunk after chunk with the whole 128 x 128 state in
//      the registers of eight wavefronts (16 columns each) -- or, for a batch
//      that would fill at most half the CUs, two workgroups of four
//      wavefronts per (sequence, v-head), half the state each; the chunk's
//      K, Q rows and slot reach LDS by DMA a chunk ahead, into the other of
//      two buffers.  Products with fp32 operands run as bf16 MFMA on hi/lo
//      splits.  Each workgroup reads its chunks' inputs once, so the
//      workspace is the only HBM traffic beyond the algorithmic bytes.
//   One long sequence at few v-heads is cut into segments, since its scan
//   alone would occupy HV workgroups for the whole run: a first scan launch
//   runs, without outputs, segment 0 from the sequence's state and, from
//   each later segment's start, the transition columns (an identity start,
//   no values) and the zero-start end state; a combine kernel chains the
//   segment starts; a second scan launch runs every segment from its start
//   with the outputs.
//
// MFMA lane layouts (v_mfma_f32_16x16x4_f32, v_mfma_f32_16x16x32_bf16):
// A[i][k] from lane i + 16 g, B[k][j] from lane j + 16 g (k = g for fp32;
// for bf16 the lane's 8 items cover the 32-long k block), D[i][j] in lane
// j + 16 (i / 4), register i % 4.  A bf16 product sums over its k block in
// any order both operands share.  Where the contracted index is a token,
// item e of lane group g stands for
//   k = 16 (e / 4) + 4 g + e % 4,
// so a lane's 8 items are the 4-element runs at k = 4 g and 16 + 4 g, the
// runs a 16 x 16 MFMA result holds per lane -- results become operands
// without exchanging data between lanes.  Where it is a key (K and Q rows
// read from LDS against the state), item e of lane group g is key 8 g + e of
// the 32-key block: one 16-byte read per operand, and the 8 lanes that the
// LDS serves together read 8 rows whose 272-byte stride puts them on
// disjoint banks.  The state's registers hold its keys in that order.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <mutex>

#include "gdn_decode_kernel.h"
#include "gdn_prefill.h"

namespace gdn_pf {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

constexpr int kDim = 128;            // K == V == 128
constexpr int kChunk = 64;           // tokens per chunk
constexpr int kThreads = 256;        // 4 wavefronts
// Batches whose chunk slots the kernels find themselves, without the offsets
// kernel: at most kFewSeqs sequences and kFewPrepGroups preparation
// workgroups (slots x v-heads).  Each workgroup then scans the batch's
// sequence lengths in one wave, which costs more than the saved launch once
// there are thousands of them (16 x 512 tokens at 16/32 heads, 4608
// workgroups: 2% slower; 8 x 1024 at 4/8, 1088: 3% faster; 3 sequences of
// 30-50 tokens: 18.7 -> 16.3 us).
constexpr int kFewSeqs = 64;
constexpr long long kFewPrepGroups = 2048;

// Chunk slots the workspace holds for L tokens in N sequences: every chunk
// of a well-formed batch fits, sum(ceil(len_i / 64)) <= ceil(L / 64) + N, and
// every chunk holds at least one token, so there are at most L of them.
// For malformed cu_seqlens the kernels cap the slots they use at this count.
long long max_slots(long long L, long long N) {
  const long long by_seqs = (L + kChunk - 1) / kChunk + N;
  return by_seqs < L ? by_seqs : L;
}

bool few_seqs(long long L, long long N, long long HV) {
  return N > 1 && N <= kFewSeqs && max_slots(L, N) * HV <= kFewPrepGroups;
}
// Total tokens up to which the token-by-token kernel runs the prefill (so no
// sequence is longer).  Measured (one sequence, calls timed from the first to
// the last event of the timed entry): the token path is 1-3.5 us faster up to
// 56 tokens at qk4_v8 and qk16_v32, the chunkwise kernels faster from 64.
// Several short sequences favour the token path far more (4 x 20 tokens: 21.2
// against 33.5 us at qk4_v8); past the switch the longest sequence is known
// only on the device (maybe_all_short below).
constexpr int kSmallTokens = 56;

// Batches of 2..kFewSeqs sequences with at most kSmallTokens tokens a
// sequence on average may have no longer sequence, which only cu_seqlens on
// the device tells: they launch the token-by-token kernel first (it runs
// only if every sequence is that short) and then the chunkwise kernels
// (which return at once in that case).  4 sequences of 20 tokens at qk4_v8
// then take the token kernel's time instead of the chunkwise kernels'.
bool maybe_all_short(long long L, long long N) {
  return L > kSmallTokens && N >= 2 && N <= kFewSeqs && L <= N * kSmallTokens;
}
constexpr float kL2Eps = 1e-6f;
// v-heads of a GVA group whose gate inputs the preparation kernel loads with
// the chunk's K rows (the others' when it reaches them).
constexpr int kPrepGateHeads = 2;
// A preparation workgroup takes a whole GVA group of v-heads (K K^T made
// once for all of them, the v-heads one after another) unless one workgroup
// per (slot, v-head) all fit on the GPU at once (4 a CU, 256 CUs): then each
// takes one v-head, and the chain of one workgroup -- the preparation's time
// on a grid that small -- is one v-head's (15k against 25k cycles at ratio 2).
constexpr long long kPrepSplitMaxWorkgroups = 1024;
inline bool prep_split(long long slots, int HV) {
  return slots * HV <= kPrepSplitMaxWorkgroups;
}
constexpr float kSoftplusThreshold = 20.0f;
constexpr float kLn2 = 0.693147180559945309f;

// Workspace slot of one (chunk, v-head), offsets in floats.  The scan's MFMA
// operand T diag(beta) is stored in operand order: a 16 x 32 block is 64
// lanes x 8 bf16 contiguous (lane = row + 16 g, items in the k order above),
// so a wave reads one with a single 1 KiB access.  It is lower triangular
// 64 x 64, so only the blocks (row block rb, token block kb) with kb <= rb / 2
// are kept, six of eight, split into a bf16 high and low part (x ~ hi + lo
// to ~2^-16 relative).  Then rows of 64 per-token scales.
constexpr int kBlk = 512;                             // bf16 per 16 x 32 operand block
constexpr int kBlkF = kBlk / 2;                       // the same in floats
constexpr int kTriBlocks = 6;
__host__ __device__ constexpr int tri_blk(int rb, int kb) { return (rb < 3 ? rb : 4) + kb; }
constexpr int kSlotTh = 0;                            // T diag(beta), hi
constexpr int kSlotTl = kSlotTh + kTriBlocks * kBlkF; //   lo
constexpr int kSlotXg = kSlotTl + kTriBlocks * kBlkF; // rk_i e^gamma_i [64]
constexpr int kSlotEg = kSlotXg + kChunk;             // e^gamma_i [64]
constexpr int kSlotKs = kSlotEg + kChunk;             // rk_i e^(gamma_C - gamma_i) [64]
constexpr int kSlotGl = kSlotKs + kChunk;             // e^gamma_C [64 copies]
constexpr int kSlotGa = kSlotGl + kChunk;             // gamma_i [64]
constexpr int kSlotRk = kSlotGa + kChunk;             // rk_i [64]
constexpr int kSlotFloats = kSlotRk + 3 * kChunk;     // padded to whole 1 KiB DMA pieces
static_assert(kSlotFloats % 256 == 0, "slots stay 1 KiB aligned");
static_assert(tri_blk(3, 1) == kTriBlocks - 1, "six lower blocks");

// Token (0..31) of item e of lane group g inside a 32-long block of a
// token-contracted operand.
__host__ __device__ constexpr int k_of(int g, int e) { return 16 * (e >> 2) + 4 * g + (e & 3); }

// First of the 4 keys that register t of a state column holds in lane group
// g (items e = 0..3 are that key + e): st[2 kb] and st[2 kb + 1] together
// are keys 32 kb + 8 g .. + 7, the key order of frag().  A 16-row key tile
// t of the state update is thus keys state_key(t, i / 4) + i % 4.
__host__ __device__ constexpr int state_key(int t, int g) {
  return 32 * (t >> 1) + 8 * g + 4 * (t & 1);
}

// LDS row strides (elements) chosen so MFMA operand reads spread over banks.
constexpr int kBfStride = kDim + 8;       // bf16 rows of 128
constexpr int kF64Stride = kChunk + 4;    // fp32 rows of 64

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Two floats to a packed bf16 pair (round to nearest even), element 0 in
// the low half.  split4: x ~ hi + lo with hi = bf16(x), lo = bf16(x - hi).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}

__device__ __forceinline__ void split4(const f32x4& x, s16x4& hi, s16x4& lo) {
  u32x2 h, l;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const float x0 = x[2 * e], x1 = x[2 * e + 1];
    h[e] = pack_bf16x2(x0, x1);
    l[e] = pack_bf16x2(x0 - __uint_as_float(h[e] << 16), x1 - __uint_as_float(h[e] & 0xffff0000u));
  }
  hi = __builtin_bit_cast(s16x4, h);
  lo = __builtin_bit_cast(s16x4, l);
}

// Workgroup barrier that orders LDS only.  The waves of these kernels
// exchange data through LDS alone, so global loads issued ahead of a barrier
// (the next chunk's operands) stay in flight across it instead of being
// drained as __syncthreads' all-memory fence would.
// The wavefront's index in its workgroup, as a value the compiler knows is
// the same in every lane (a scalar register): branches on it are scalar
// branches and LDS bases derived from it need no per-lane waterfall.  Used by
// the scan (64 x 512 qk16_v32: scan 485.9 -> 457.8 us with the L2-norm as a
// template flag); the preparation kernel keeps threadIdx.x >> 6, with which
// it measured faster (118.8 against 138.9 us).
__device__ __forceinline__ int wave_index() {
  return __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
}

__device__ __forceinline__ void block_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ f32x4 mfma_f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_bf16(s16x8 a, s16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ s16x8 cat(s16x4 a, s16x4 b) {
  return s16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// Operand items of lane group g for key block kb of a bf16 row of 128 keys
// in LDS: keys 32 kb + 8 g .. + 7, one 16-byte read (rows 16-byte aligned).
__device__ __forceinline__ s16x8 frag(const uint16_t* row, int kb, int g) {
  return *reinterpret_cast<const s16x8*>(row + 32 * kb + 8 * g);
}

struct Params {
  const uint16_t* q;         // [L, H, 128] bf16
  const uint16_t* k;         // [L, H, 128] bf16
  const uint16_t* v;         // [L, HV, 128] bf16
  const float* state;        // [N, HV, 128, 128] fp32 k-last, or null (zeros)
  const float* A_log;        // [HV]
  const uint16_t* a;         // [L, HV] bf16
  const float* dt_bias;      // [HV]
  const uint16_t* b;         // [L, HV] bf16
  const int32_t* cu_seqlens; // [N + 1]
  uint16_t* out;             // [L, HV, 128] bf16
  float* new_state;          // [N, HV, 128, 128] fp32 k-last
  const int32_t* offs;       // [N + 1] first chunk slot of each sequence (workspace)
  const i32x4* slot_info;    // [max_slots] per chunk slot: sequence, first token, tokens
                             // (0 past the last slot) (workspace)
  float* slots;              // [max_slots, HV, kSlotFloats] (workspace)
  float scale;
  int L;
  int N;
  int H;
  int HV;
  int ratio;                 // HV / H
  int l2norm;
  int single;                // one sequence: chunk c is slot c (no offsets kernel)
  int few;                   // 2..kFewSeqs sequences: the kernels compute the chunk
                             // slots from cu_seqlens (no offsets kernel)
  long long max_slots;       // slots the workspace holds
  // Segments (seg_chunks > 0): segment j of a sequence is its chunks
  // [j seg_chunks, (j + 1) seg_chunks), and the segments of all sequences are
  // numbered in sequence order (at most nseg); per (segment, v-head) 128 x 128 fp32
  // blocks in k-last order (element (k, c) at c * 128 + k).
  int seg_chunks;            // chunks per segment, 0: no segments
  int nseg;                  // segments
  float* seg_S;              // [nseg, HV] state at each segment's start (1 .. nseg-1)
  float* seg_B;              // [nseg, HV] state at its end from a zero start
  float* seg_M;              // [nseg, HV] its transition: end = M start + B (M[k][k'])
  // > 0: the token-by-token kernel was launched first with this limit (at
  // most kFewSeqs sequences); if every sequence has at most this many tokens
  // it ran the whole prefill and these kernels return at once.
  int short_limit;
  int prep_heads;            // v-heads per preparation workgroup: ratio, or 1
};

// Token range [start, end) of sequence s, clamped to [0, L] so that no
// cu_seqlens content makes a kernel read outside the inputs.
__device__ __forceinline__ void seq_range(const Params& p, int s, int& start, int& end) {
  int s0 = p.cu_seqlens[s];
  int s1 = p.cu_seqlens[s + 1];
  s0 = s0 < 0 ? 0 : (s0 > p.L ? p.L : s0);
  s1 = s1 < s0 ? s0 : (s1 > p.L ? p.L : s1);
  start = s0;
  end = s1;
}

// Whether every sequence of a batch of at most 64 has at most `limit`
// tokens (one read per lane, the clamping of seq_range; uniform).
__device__ __forceinline__ bool all_within(const Params& p, int limit) {
  const int lane = threadIdx.x & 63;
  int len = 0;
  if (lane < p.N) {
    int s0, s1;
    seq_range(p, lane, s0, s1);
    len = s1 - s0;
  }
  return __ballot(len > limit) == 0;
}

// Chunk slots of a batch of at most 64 sequences, from cu_seqlens in one
// wave (lane s: sequence s): the prefix the offsets kernel writes, held in
// registers.  excl = slots of the sequences before s, incl = excl + its own,
// both capped at the workspace's slots as there.  A sequence's chunk count
// is at most 2^25 (ranges are clamped to [0, L], L < 2^31), so 64 of them
// sum without overflow in 32 bits.
struct FewSlots {
  int start, end;          // this lane's sequence's token range (0, 0 past N)
  long long excl, incl;
};

__device__ __forceinline__ FewSlots few_slots(const Params& p) {
  const int lane = threadIdx.x & 63;
  FewSlots f{0, 0, 0, 0};
  unsigned cnt = 0;
  if (lane < p.N) {
    seq_range(p, lane, f.start, f.end);
    cnt = static_cast<unsigned>(f.end - f.start + kChunk - 1) / kChunk;
  }
  unsigned x = cnt;                                // inclusive scan over the wave
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const unsigned y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  const long long incl = x, excl = static_cast<long long>(x) - cnt;
  f.incl = incl < p.max_slots ? incl : p.max_slots;
  f.excl = excl < p.max_slots ? excl : p.max_slots;
  return f;
}

// Segments of a batch of at most 64 sequences, in one wave (lane s: sequence
// s): its token range, its segment count (seg_chunks chunks a segment; one
// for an empty sequence), the segments of the sequences before it, and its
// units of a segment launch (OUT: one a segment; else 2 nseg - 3: segment 0
// from the sequence's state, the middle ones from a zero start and from the
// identity; none for a sequence of one segment).
struct SegSeqs {
  int start, end;
  int nseg, seg_excl;
  int u_excl, u_incl;
};

// Units of the first segment launch for nseg segments in all: one sequence
// has 2 nseg - 3, several at most 2 nseg.
__host__ __device__ inline long long seg_units1(long long nseg, long long N) {
  return N == 1 ? 2 * nseg - 3 : 2 * nseg;
}

template <bool OUT>
__device__ __forceinline__ SegSeqs seg_seqs(const Params& p) {
  const int lane = threadIdx.x & 63;
  SegSeqs f{0, 0, 0, 0, 0, 0};
  int units = 0;
  if (lane < p.N) {
    seq_range(p, lane, f.start, f.end);
    const int nch = (f.end - f.start + kChunk - 1) / kChunk;
    f.nseg = nch > p.seg_chunks ? (nch + p.seg_chunks - 1) / p.seg_chunks : 1;
    units = OUT ? f.nseg : (f.nseg >= 2 ? 2 * f.nseg - 3 : 0);
  }
  if (p.N == 1) {                                  // uniform: nothing to scan
    f.u_incl = units;
    return f;
  }
  int xs = f.nseg, xu = units;                     // inclusive scans over the wave
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int ys = __shfl_up(xs, d, 64);
    const int yu = __shfl_up(xu, d, 64);
    if (lane >= d) {
      xs += ys;
      xu += yu;
    }
  }
  f.seg_excl = xs - f.nseg;
  f.u_excl = xu - units;
  f.u_incl = xu;
  // A malformed batch (overlapping ranges) may need more segments than the
  // workspace holds: then every sequence is one segment (a plain scan in the
  // second launch), so each one's state is still written.
  if (__builtin_amdgcn_readlane(xs, 63) > p.nseg) {
    f.nseg = lane < p.N ? 1 : 0;
    f.seg_excl = lane;
    f.u_excl = OUT ? lane : 0;
    f.u_incl = OUT && lane < p.N ? lane + 1 : f.u_excl;
  }
  return f;
}

// ---------------------------------------------------------------------------
// 1. chunk slots per sequence
// ---------------------------------------------------------------------------
// One workgroup of 256 threads: each thread counts one sequence's chunks, a
// block-wide inclusive scan (wave scans through LDS) turns 256 counts into
// offsets, and a running total carries from one group of 256 sequences to
// the next.  The group's offsets and token ranges then go to LDS, and the
// threads fill the group's slots of the slot table, each finding its slot's
// sequence by binary search there.  Slots past the last one get zero tokens.
__global__ __launch_bounds__(kThreads) void chunk_offsets_kernel(Params p, int32_t* offs,
                                                                 i32x4* slot_info) {
  __shared__ long long wave_sum[kThreads / 64];
  __shared__ int32_t grp_offs[kThreads + 1];   // offs[base .. base + 256]
  __shared__ int32_t grp_start[kThreads];
  __shared__ int32_t grp_end[kThreads];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  if (p.short_limit > 0 && all_within(p, p.short_limit)) return;    // uniform
  long long carry = 0;
  if (threadIdx.x == 0) offs[0] = 0;
  for (int base = 0; base < p.N; base += kThreads) {
    const int s = base + threadIdx.x;
    long long cnt = 0;
    int start = 0, end = 0;
    if (s < p.N) {
      seq_range(p, s, start, end);
      cnt = (end - start + kChunk - 1) / kChunk;
    }
    long long x = cnt;                         // inclusive scan within the wave
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const long long y = __shfl_up(x, d, 64);
      if (lane >= d) x += y;
    }
    if (lane == 63) wave_sum[wave] = x;
    __syncthreads();
    long long before = carry;
    for (int w = 0; w < wave; ++w) before += wave_sum[w];
    long long total = carry;
    for (int w = 0; w < kThreads / 64; ++w) total += wave_sum[w];
    long long v = before + x;
    if (v > p.max_slots) v = p.max_slots;      // only for overlapping ranges
    if (total > p.max_slots) total = p.max_slots;
    if (s < p.N) offs[s + 1] = static_cast<int32_t>(v);
    grp_offs[threadIdx.x + 1] = static_cast<int32_t>(v);
    if (threadIdx.x == 0) grp_offs[0] = static_cast<int32_t>(carry);
    grp_start[threadIdx.x] = start;
    grp_end[threadIdx.x] = end;
    carry = total;
    __syncthreads();
    // slots [grp_offs[0], grp_offs[256]) belong to this group's sequences;
    // slot c's sequence is the largest j with grp_offs[j] <= c
    for (int c = grp_offs[0] + threadIdx.x; c < grp_offs[kThreads]; c += kThreads) {
      int lo = 0, hi = kThreads - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (grp_offs[mid] <= c) lo = mid; else hi = mid - 1;
      }
      const int t0 = grp_start[lo] + (c - grp_offs[lo]) * kChunk;
      const int n = min(kChunk, grp_end[lo] - t0);
      slot_info[c] = i32x4{base + lo, t0, n, 0};
    }
    __syncthreads();                           // LDS is rewritten next round
  }
  for (long long c = carry + threadIdx.x; c < p.max_slots; c += kThreads)
    slot_info[c] = i32x4{0, 0, 0, 0};
}

// Gates of token t, v-head hv: log-space decay and beta
// (g = exp(-exp(A_log) softplus(a + dt_bias)), beta = sigmoid(b)).
__device__ __forceinline__ void gates_of(uint16_t a_raw, uint16_t b_raw, float dt_bias,
                                         float A_log, float& logg, float& beta) {
  const float x = bf16_to_f32(a_raw) + dt_bias;
  const float sp = x > kSoftplusThreshold ? x : __builtin_amdgcn_logf(1.0f + __expf(x)) * kLn2;
  logg = -__expf(A_log) * sp;
  beta = __builtin_amdgcn_rcpf(1.0f + __expf(-bf16_to_f32(b_raw)));
}

__device__ __forceinline__ void token_gates(const Params& p, int t, int hv, float& logg,
                                            float& beta) {
  gates_of(p.a[static_cast<size_t>(t) * p.HV + hv], p.b[static_cast<size_t>(t) * p.HV + hv],
           p.dt_bias[hv], p.A_log[hv], logg, beta);
}

// One DPP step of a wave scan: x from the lane CTRL names (0 where it names
// none, or in rows ROW_MASK leaves out).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add_src(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x),
                                                               CTRL, ROW_MASK, 0xf, false));
}

// Inclusive prefix sum over the 64 lanes of a wave: shifts by 1, 2, 4 and 8
// within each row of 16 lanes (row_shr), then lane 15's total added to rows
// 1 and 3 and lane 31's to rows 2 and 3 (row_bcast:15, row_bcast:31).
__device__ __forceinline__ float wave_prefix_sum(float x) {
  x += dpp_add_src<0x111, 0xf>(x);
  x += dpp_add_src<0x112, 0xf>(x);
  x += dpp_add_src<0x114, 0xf>(x);
  x += dpp_add_src<0x118, 0xf>(x);
  x += dpp_add_src<0x142, 0xa>(x);
  x += dpp_add_src<0x143, 0xc>(x);
  return x;
}

// Rows [0, 64) of a [*, stride, 128] bf16 tensor (row r at base + r * step
// elements) as 4 pieces of 16 bytes per thread.  Rows >= n read row n - 1
// (n >= 1) so that every load is unconditional: issued together, waited on
// once.  store_rows_bf16 writes them to LDS rows of kBfStride, zeroing rows
// >= n.
__device__ __forceinline__ void load_rows_bf16(u32x4 (&val)[4], const uint16_t* base,
                                               size_t step, int n) {
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int idx = threadIdx.x + it * kThreads;
    const int r = idx >> 4;
    const int rr = r < n ? r : n - 1;
    val[it] = *reinterpret_cast<const u32x4*>(base + static_cast<size_t>(rr) * step +
                                              (idx & 15) * 8);
  }
}

__device__ __forceinline__ void store_rows_bf16(uint16_t* dst, const u32x4 (&val)[4], int n) {
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int idx = threadIdx.x + it * kThreads;
    const int r = idx >> 4;
    const u32x4 x = r < n ? val[it] : u32x4{0u, 0u, 0u, 0u};
    uint16_t* d = dst + r * kBfStride + (idx & 15) * 8;
    *reinterpret_cast<u32x2*>(d) = u32x2{x.x, x.y};
    *reinterpret_cast<u32x2*>(d + 4) = u32x2{x.z, x.w};
  }
}

// ---------------------------------------------------------------------------
// 2. per-chunk preparation
// ---------------------------------------------------------------------------

// 35 KiB, so that four workgroups share a CU: A takes the place of the K
// rows, which no wave reads once K K^T is in registers (every wave passes a
// barrier between its last K read and the first write of A).  The 32 x 32
// scratch of the block recursion is T's upper-right quarter, which T never
// uses (rows 0..31, columns 32..63).
struct __attribute__((aligned(16))) PrepLds {
  union {
    uint16_t K[kChunk * kBfStride];   // the chunk's K rows, until K K^T
    float A[kChunk * kF64Stride];     // then: strict lower part of (I + A) minus I
  };
  float T[kChunk * kF64Stride];       // (I + A)^-1
  float gamma[kChunk];
  float beta[kChunk];
  float rk[kChunk];
};
static_assert(sizeof(PrepLds) <= 160 * 1024 / 4, "four preparation workgroups per CU");

// 16 x 16 x 16 fp32 block product A[0:16, 0:16] B[0:16, 0:16] from LDS rows
// of stride lda / ldb, as an MFMA result (lane (col, g) holds rows 4 g + e).
__device__ __forceinline__ f32x4 mm16_f32(const float* A, int lda, const float* B, int ldb,
                                          int col, int g4) {
  f32x4 acc = {0, 0, 0, 0};
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
    acc = mfma_f32(A[col * lda + 4 * ks + g4], B[(4 * ks + g4) * ldb + col], acc);
  return acc;
}

__device__ __forceinline__ void store16(float* D, int ldd, const f32x4& v, float sign, int col,
                                        int g4) {
#pragma unroll
  for (int e = 0; e < 4; ++e) D[(4 * g4 + e) * ldd + col] = sign * v[e];
}

// One chunk's preparation, tokens t0 .. t0 + n - 1 (n: 1..64) of q/k head h,
// for v-heads hv0 .. hv0 + prep_heads - 1, by the 256 threads of the calling
// workgroup: the slots go to the workspace (slot c), or with LDS_SLOT (one
// v-head) to lds_slot in the calling workgroup's LDS.
template <bool LDS_SLOT>
__device__ __forceinline__ void prep_chunk(Params p, int c, int t0, int n, int hv0, int h,
                                           int prep_heads, PrepLds& lds, float* lds_slot) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int col = lane & 15;
  const int g4 = lane >> 4;

  // Every input load of the chunk is issued before the first is waited on.
  u32x4 kreg[4];
  load_rows_bf16(kreg, p.k + (static_cast<size_t>(t0) * p.H + h) * kDim,
                 static_cast<size_t>(p.H) * kDim, n);
  // wave 0's gate inputs (a, b of token t0 + lane) of the group's first
  // kPrepGateHeads v-heads, in flight with the K rows
  uint16_t a_raw[kPrepGateHeads], b_raw[kPrepGateHeads];
  float dtb[kPrepGateHeads], alog[kPrepGateHeads];
  if (wave == 0) {
    const size_t tk = static_cast<size_t>(t0 + (lane < n ? lane : n - 1)) * p.HV + hv0;
#pragma unroll
    for (int j = 0; j < kPrepGateHeads; ++j) {
      const int jj = j < prep_heads ? j : 0;
      a_raw[j] = p.a[tk + jj];
      b_raw[j] = p.b[tk + jj];
      dtb[j] = p.dt_bias[hv0 + jj];
      alog[j] = p.A_log[hv0 + jj];
    }
  }

  store_rows_bf16(lds.K, kreg, n);
  // T's upper blocks that the block recursion multiplies, T_01 and T_23, are
  // zero; the diagonal and lower blocks are all written, the other upper
  // blocks never read.
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int idx = threadIdx.x + it * kThreads;
    const int o = 32 * (idx >> 8);
    lds.T[(o + ((idx >> 4) & 15)) * kF64Stride + o + 16 + (idx & 15)] = 0.0f;
  }
  block_sync_lds();

  // K row scales of the L2-norm (1 when off): 4 threads per row.
  {
    const int r = threadIdx.x >> 2;
    const int part = threadIdx.x & 3;
    float sk = 0.0f;
    if (p.l2norm) {
      for (int i = part * 32; i < part * 32 + 32; ++i) {
        const float y = bf16_to_f32(lds.K[r * kBfStride + i]);
        sk = fmaf(y, y, sk);
      }
      sk += __shfl_xor(sk, 1, 64);
      sk += __shfl_xor(sk, 2, 64);
    }
    if (part == 0) lds.rk[r] = p.l2norm ? __builtin_amdgcn_rsqf(sk + kL2Eps) : 1.0f;
  }
  block_sync_lds();

  // K K^T for row block `wave` (rows 16 wave .. +15), column blocks 0 ..
  // wave (A is strictly lower triangular: the blocks right of the diagonal
  // are neither computed nor written); bf16 MFMA over the 128-long rows
  f32x4 kk[4];
  {
#pragma unroll
    for (int nj = 0; nj < 4; ++nj) kk[nj] = f32x4{0, 0, 0, 0};
    const int ra = wave * 16 + col;
#pragma unroll
    for (int m = 0; m < kDim / 32; ++m) {
      const s16x8 ak = frag(&lds.K[ra * kBfStride], m, g4);
#pragma unroll
      for (int nj = 0; nj < 4; ++nj) {
        if (nj > wave) break;                      // uniform per wave
        const s16x8 bk = frag(&lds.K[(nj * 16 + col) * kBfStride], m, g4);
        kk[nj] = mfma_bf16(ak, bk, kk[nj]);
      }
    }
  }

  // Each v-head of the group: its gates, A from the shared product, T, and
  // its slot.  The LDS the previous v-head used (gamma, beta, A, T)
  // is rewritten only after the barrier that ends its use.
  for (int j = 0; j < prep_heads; ++j) {
    const int hv = hv0 + j;
    float* slot = LDS_SLOT ? lds_slot
                           : p.slots + (static_cast<size_t>(c) * p.HV + hv) * kSlotFloats;
    uint16_t* slot16 = reinterpret_cast<uint16_t*>(slot);
    // gates of token t0 + lane (padded rows: no decay, no update), and the
    // inclusive scan of the log-decay over the chunk
    if (wave == 0) {
      float logg, beta;
      if (j < kPrepGateHeads) {
        uint16_t ar = a_raw[0], br = b_raw[0];
        float dt = dtb[0], al = alog[0];
#pragma unroll
        for (int jj = 1; jj < kPrepGateHeads; ++jj)
          if (j == jj) { ar = a_raw[jj]; br = b_raw[jj]; dt = dtb[jj]; al = alog[jj]; }
        gates_of(ar, br, dt, al, logg, beta);
      } else {
        token_gates(p, t0 + (lane < n ? lane : n - 1), hv, logg, beta);
      }
      if (lane >= n) logg = beta = 0.0f;
      lds.gamma[lane] = wave_prefix_sum(logg);
      lds.beta[lane] = beta;
    }
    block_sync_lds();
    {
      // Row and column factors, read once.  The decays are computed for every
      // element with the exponent clamped to <= 0 (it is <= 0 wherever the
      // element is kept: gamma does not increase) and the masks are selects.
      // A[i][j], i = 16 wave + 4 g + e, j = 16 nj + col (K K^T is symmetric)
      const int ia = wave * 16 + g4 * 4;
      const f32x4 gi4 = *reinterpret_cast<const f32x4*>(&lds.gamma[ia]);
      const f32x4 bri4 = *reinterpret_cast<const f32x4*>(&lds.beta[ia]) *
                         *reinterpret_cast<const f32x4*>(&lds.rk[ia]);
#pragma unroll
      for (int nj = 0; nj < 4; ++nj) {
        if (nj > wave) break;                      // uniform: never read
        const int j = nj * 16 + col;
        const float gj = lds.gamma[j];
        const float rkj = lds.rk[j];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float dec = __expf(fminf(gi4[e] - gj, 0.0f));
          const float x = bri4[e] * rkj * dec * kk[nj][e];
          lds.A[(ia + e) * kF64Stride + j] = j < ia + e ? x : 0.0f;
        }
      }
    }
    block_sync_lds();

    // T = (I + A)^-1 by block recursion on 16 x 16 blocks (A is strictly lower
    // triangular, so T is unit lower triangular; the upper blocks stay zero):
    // 1. each wave inverts one diagonal block by forward substitution (one
    //    column per lane, two partial sums per dot product);
    //    Row r's entries of A are read as 16-byte vectors a row ahead of
    //    their use (read when used, their LDS latency was most of the
    //    substitution's).
    if (lane < 16) {
      const int b0 = wave * 16;
      const float* arow = &lds.A[b0 * kF64Stride + b0];
      float t[16];
      f32x4 ar[16][4];
      auto read_row = [&](int r) {
#pragma unroll
        for (int q = 0; q < (r + 3) / 4; ++q)
          ar[r][q] = *reinterpret_cast<const f32x4*>(&arow[r * kF64Stride + 4 * q]);
      };
      read_row(1);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        if (r + 1 < 16) read_row(r + 1);
        float s0 = (r == lane) ? 1.0f : 0.0f, s1 = 0.0f;
#pragma unroll
        for (int j = 0; j < r; ++j) {
          const float aij = ar[r][j >> 2][j & 3];
          if (j & 1) s1 = fmaf(-aij, t[j], s1); else s0 = fmaf(-aij, t[j], s0);
        }
        t[r] = s0 + s1;
        lds.T[(b0 + r) * kF64Stride + b0 + lane] = t[r];
      }
    }
    block_sync_lds();
    // 2. the 32 x 32 diagonal halves: T_10 = -T_11 A_10 T_00 (wave 0) and
    //    T_32 = -T_33 A_32 T_22 (wave 1), through LDS within the wave;
    if (wave < 2) {
      const int b = wave * 32;
      float* Xw = &lds.T[32] + wave * 16 * kF64Stride;
      const f32x4 x = mm16_f32(&lds.A[(b + 16) * kF64Stride + b], kF64Stride,
                               &lds.T[b * kF64Stride + b], kF64Stride, col, g4);
      store16(Xw, kF64Stride, x, 1.0f, col, g4);
      const f32x4 y = mm16_f32(&lds.T[(b + 16) * kF64Stride + b + 16], kF64Stride, Xw,
                               kF64Stride, col, g4);
      store16(&lds.T[(b + 16) * kF64Stride + b], kF64Stride, y, -1.0f, col, g4);
    }
    block_sync_lds();
    // 3. the lower-left 32 x 32 quarter: T_BA = -T_B (A_BA T_A), one 16 x 16
    //    tile per wave.
    {
      const int rb = wave >> 1, cb = wave & 1;
      const float* Arow = &lds.A[(32 + 16 * rb) * kF64Stride];
      const f32x4 x = mm16_f32(Arow, kF64Stride, &lds.T[16 * cb], kF64Stride, col, g4) +
                      mm16_f32(Arow + 16, kF64Stride, &lds.T[16 * kF64Stride + 16 * cb],
                               kF64Stride, col, g4);
      store16(&lds.T[16 * rb * kF64Stride + 32 + 16 * cb], kF64Stride, x, 1.0f, col, g4);
    }
    block_sync_lds();
    {
      const int rb = wave >> 1, cb = wave & 1;
      const float* Trow = &lds.T[(32 + 16 * rb) * kF64Stride + 32];
      const float* X = &lds.T[32];
      const f32x4 y = mm16_f32(Trow, kF64Stride, &X[16 * cb], kF64Stride, col, g4) +
                      mm16_f32(Trow + 16, kF64Stride, &X[16 * kF64Stride + 16 * cb], kF64Stride,
                               col, g4);
      store16(&lds.T[(32 + 16 * rb) * kF64Stride + 16 * cb], kF64Stride, y, -1.0f, col, g4);
    }
    block_sync_lds();

    // T diag(beta) in operand order: lower block (rb, kb) holds, for lane
    // (col, g), T[16 rb + col][32 kb + k] beta[32 kb + k] at the 8 k of its
    // items.  Wave w writes block w, waves 0 and 1 also blocks 4 and 5.
    // Blocks (0, 0) and (2, 1) read T_01 and T_23 (zero); none reads the
    // recursion's scratch quarter.
#pragma unroll
    for (int rep = 0; rep < 2; ++rep) {
      const int idx = wave + 4 * rep;
      if (idx >= kTriBlocks) break;                  // uniform per wave
      const int rb = idx < 3 ? idx : (idx + 2) >> 1;     // tri_blk(rb, kb) == idx
      const int kb = idx == 3 || idx == 5 ? 1 : 0;
      const float* trow = &lds.T[(16 * rb + col) * kF64Stride + 32 * kb + 4 * g4];
      const float* brow = &lds.beta[32 * kb + 4 * g4];
      s16x4 hi[2], lo[2];
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
        split4(*reinterpret_cast<const f32x4*>(trow + 16 * hf) *
                   *reinterpret_cast<const f32x4*>(brow + 16 * hf),
               hi[hf], lo[hf]);
      const int bo = idx * kBlk + lane * 8;
      *reinterpret_cast<s16x8*>(slot16 + 2 * kSlotTh + bo) = cat(hi[0], hi[1]);
      *reinterpret_cast<s16x8*>(slot16 + 2 * kSlotTl + bo) = cat(lo[0], lo[1]);
    }

    // Row scales for the scan: the decayed K rows of X, the decay of the
    // output's rows, the K rows of the state update, the chunk decay, and
    // gamma and the K row scales for its P.
    if (wave == 1) {
      const float gl = lds.gamma[kChunk - 1];        // padded rows carry gamma forward
      const float gi = lds.gamma[lane];
      const float rki = lds.rk[lane];
      const float egi = __expf(gi);
      slot[kSlotXg + lane] = rki * egi;
      slot[kSlotEg + lane] = egi;
      slot[kSlotKs + lane] = rki * __expf(gl - gi);
      slot[kSlotGl + lane] = __expf(gl);
      slot[kSlotGa + lane] = gi;
      slot[kSlotRk + lane] = rki;
    }
    block_sync_lds();                        // this v-head's LDS reads are done
  }
}

// FEW: the batch's chunk slots come from cu_seqlens in the kernel (few
// sequences, no offsets kernel); a template flag, so that the kernels of the
// other modes are compiled without that code.
template <bool FEW>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4)))
void prep_kernel(Params p) {
  __shared__ PrepLds lds;
  const int c = blockIdx.x;
  // v-heads hv0 .. hv0 + prep_heads - 1, all of q/k head h
  const int hv0 = static_cast<int>(blockIdx.y) * p.prep_heads;
  const int h = hv0 / p.ratio;
  if (p.short_limit > 0 && all_within(p, p.short_limit)) return;    // uniform
  int t0, n;                                       // n: 1..64, 0 past the last slot
  if (p.single) {
    int start, end;
    seq_range(p, 0, start, end);
    t0 = start + c * kChunk;
    n = min(kChunk, end - t0);
  } else if (FEW) {
    // slot c belongs to the sequence whose slots [excl, incl) hold it
    const FewSlots f = few_slots(p);
    const unsigned long long own = __ballot(f.excl <= c && c < f.incl);
    t0 = 0;
    n = 0;
    if (own != 0) {
      const int s = __builtin_ctzll(own);
      const long long first = __shfl(f.excl, s, 64);
      t0 = __shfl(f.start, s, 64) + static_cast<int>(c - first) * kChunk;
      n = min(kChunk, __shfl(f.end, s, 64) - t0);
    }
  } else {
    const i32x4 info = p.slot_info[c];
    t0 = info.y;
    n = info.z;
  }
  if (n <= 0) return;                              // uniform per workgroup
  prep_chunk<false>(p, c, t0, n, hv0, h, p.prep_heads, lds, nullptr);
}

// ---------------------------------------------------------------------------
// 3. the scan: one workgroup per (sequence, v-head) and the whole state, or
//    two per (sequence, v-head) and half the state each
// ---------------------------------------------------------------------------
// W waves (8, two per SIMD; or 4, one per SIMD): the wave of column wave w
// keeps state columns 16 w .. 16 w + 15 of all 128 keys in registers, st[t]
// holding keys state_key(t, g) + e of column 16 w + col (lane (col, g)).
// Read as pairs (st[2 kb], st[2 kb + 1]: keys 32 kb + 8 g .. + 7), the same
// registers are the state's operand of a product over keys in either role
// (B of K S, A of S^T Q^T), in the key order of the K and Q operands read
// from LDS, and every per-chunk result is the next product's operand in
// place.  Per chunk, with S its start state:
//   X      = V - diag(rk e^gamma) K S
//   Delta  = T diag(beta) X
//   O^T    = S^T Q^T diag(scale rq e^gamma) + Delta^T P^T
//   S     <- e^gamma_C S + K^T diag(rk e^(gamma_C - gamma)) Delta
// as bf16 MFMA (16x16x32): K, Q, V are bf16; S, X, Delta, T diag(beta) and
// P enter split into hi + lo, and a product x y is hi_x hi_y + hi_x lo_y +
// lo_x hi_y (the lo lo term is ~2^-16 relative and dropped).
//
// The waves share the chunk's K rows, Q rows and workspace slot, which the
// LDS DMA (global_load_lds_dwordx4: each lane's 16 bytes land at the wave's
// LDS base + 16 lane, no registers) brings into one of two LDS buffers while
// the chunk before runs on the other.  The operands with tokens as the
// contracted index come from products with a selector (a 32 x 16 block of
// the identity), which moves a 16 x 32 row block's columns into the result
// layout exactly: V^T tiles (each wave's own 16 columns of V, loaded into
// registers a chunk ahead) and K^T tiles (wave w makes key tiles w, w + W,
// ... from the K rows in LDS and shares them through LDS: a second barrier
// per chunk, before the state update).
constexpr int kScanWaves = 8;
constexpr int kScanThreads = 64 * kScanWaves;
// A scan workgroup of W waves holds 16 W state columns: W = 8, the whole
// state, or W = 4, half of it (columns 64 half .. + 63), two workgroups per
// (sequence, v-head).  A workgroup holds a CU alone (its LDS), so with W = 4
// each SIMD runs one wave instead of two: a chunk step costs about half
// (its instruction issue, which the two waves of a SIMD share, sets it), for
// twice the workgroups -- the form for batches whose whole-state workgroups
// would fill at most half the CUs.
constexpr int kRowPieces = kDim / 8 + 1;          // 16-byte pieces per K / Q row, one of padding
constexpr int kRowStride = kRowPieces * 8;        // bf16 (68 dwords)
constexpr int kRowDma = kChunk * kRowPieces / 64; // DMA instructions per K / Q chunk (17)
constexpr int kSlotDma = kSlotFloats / 4 / 64;    // DMA instructions per slot (14)
static_assert(kChunk * kRowPieces % 64 == 0 && kSlotFloats % 256 == 0, "whole DMA instructions");
// K^T operand blocks of a chunk: (key tile t, token block kb), 64 lanes x 8 bf16
constexpr int kKtElems = 8 * 2 * 64 * 8;
// P' operand blocks (the six lower (row block, token block) ones), hi then lo
constexpr int kPElems = 2 * kTriBlocks * kBlk;

// 16-byte aligned: the scan reads its row scales as 16-byte vectors.
template <bool OUT> struct ScanBuf;
template <> struct __attribute__((aligned(16))) ScanBuf<true> {
  uint16_t Kr[kChunk * kRowStride];
  uint16_t Qr[kChunk * kRowStride];
  float slot[kSlotFloats];
};
template <> struct __attribute__((aligned(16))) ScanBuf<false> {  // without outputs: no Q
  uint16_t Kr[kChunk * kRowStride];
  float slot[kSlotFloats];
};
static_assert(2 * sizeof(ScanBuf<true>) + 2 * (kKtElems + kPElems) <= 160 * 1024,
              "one scan workgroup per CU");

typedef __attribute__((address_space(1))) void global_void;
typedef __attribute__((address_space(3))) void lds_void;

// One wave's DMA instruction: lane l's 16 bytes from src_l to dst + 16 l
// (dst the same for the whole wave).
__device__ __forceinline__ void dma16(const void* src_l, void* dst) {
  __builtin_amdgcn_global_load_lds((global_void*)src_l, (lds_void*)dst, 16, 0, 0);
}

// The same from a workgroup-uniform base and a 32-bit byte offset per lane:
// the address form of the instruction with the base in scalar registers, so
// no lane forms a 64-bit address.
__device__ __forceinline__ void dma16_at(const void* base, unsigned byte_off, void* dst) {
  dma16(static_cast<const char*>(base) + byte_off, dst);
}

// Byte offset of element `item` of token row `row` (< 64) of a bf16 matrix
// whose rows are `step` (< 2^24) elements apart: a 24-bit product, one
// full-rate instruction where a 32-bit one takes four.
__device__ __forceinline__ unsigned row_bytes(int row, unsigned step, unsigned item) {
  return 2u * (__umul24(static_cast<unsigned>(row), step) + item);
}

// Wait for this wave's outstanding vector memory operations (its DMA among
// them): s_waitcnt vmcnt(0), the other counters left alone.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Workgroup barrier after this wave's LDS reads and writes (s_waitcnt
// lgkmcnt(0)) but not its DMA: a fence on LDS would wait for the DMA in
// flight too (it writes LDS), which only the next chunk reads.  The empty
// asm statements keep the compiler from moving memory accesses across.
__device__ __forceinline__ void barrier_lds_no_dma() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// DMA of a chunk's K rows, Q rows (OUT; rows >= n repeat row n - 1; each
// row's padding piece repeats its last piece) and slot (SLOT) into one LDS
// buffer; wave w of W issues instructions w, w + W, ....
template <bool OUT, int W, bool SLOT = true>
__device__ __forceinline__ void scan_dma(ScanBuf<OUT>& B, const uint16_t* kbase,
                                         const uint16_t* qbase, unsigned step, int n,
                                         const float* slot, int wave, int lane) {
  for (int i = wave; i < kRowDma; i += W) {                 // uniform per wave
    const int pc = i * 64 + lane;
    const int r = pc / kRowPieces, c = pc % kRowPieces;
    const unsigned off = row_bytes(r < n ? r : n - 1, step, (c < 16 ? c : 15) * 8);
    dma16_at(kbase, off, &B.Kr[i * 512]);
    if constexpr (OUT) dma16_at(qbase, off, &B.Qr[i * 512]);
  }
  if constexpr (SLOT) {
    for (int i = wave; i < kSlotDma; i += W)
      dma16_at(slot, static_cast<unsigned>(i * 64 + lane) * 16u, &B.slot[i * 256]);
  }
}

// This wave's 16 columns of V for token tile r (lane (col, g): token
// 16 r + col, columns 16 cw + 4 g .. + 3, cw the wave's column wave; rows
// >= n repeat row n - 1).
__device__ __forceinline__ void load_v(u32x2 (&f)[4], const uint16_t* vbase, unsigned step, int n,
                                       int cw, int col, int g4) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int row = r * 16 + col;
    f[r] = *reinterpret_cast<const u32x2*>(
        reinterpret_cast<const char*>(vbase) + row_bytes(row < n ? row : n - 1, step,
                                                         cw * 16 + g4 * 4));
  }
}

__device__ __forceinline__ s16x8 split_hi_lo(const f32x4& a, const f32x4& b, s16x8& lo) {
  s16x4 ha, la, hb, lb;
  split4(a, ha, la);
  split4(b, hb, lb);
  lo = cat(la, lb);
  return cat(ha, hb);
}

__device__ __forceinline__ s16x8 ld_op(const void* ptr) {
  return *reinterpret_cast<const s16x8*>(ptr);
}

// bf16 values held in fp32 back to bf16 (exact), 4 at a time.
__device__ __forceinline__ s16x4 to_bf16x4(const f32x4& x) {
  const u32x2 w = {pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3])};
  return __builtin_bit_cast(s16x4, w);
}

// The per-workgroup constants of a scan.
struct ScanCtx {
  const uint16_t* k;
  const uint16_t* q;
  const uint16_t* v;
  uint16_t* out;
  const float* slot_base;      // the first chunk's slot
  size_t slot_step;            // floats from one chunk's slot to the next
  unsigned kstep, vstep;       // elements from one token's K / Q row (V row) to the next
  int start, end, nchunks;     // token range and chunks
  int H, HV, h, hv;
  float scale;
  bool values;
  int cw0;                     // the first wave's column wave: 0, or 4 for the second half
};

// Column wave of wave `wave` (columns 16 cw .. 16 cw + 15): with W = 8 the
// wave itself (cw0 is 0; known here at compile time).
template <int W>
__device__ __forceinline__ int column_wave(const ScanCtx& cx, int wave) {
  return W == kScanWaves ? wave : cx.cw0 + wave;
}

// Chunk c's DMA into buf (its slot with SLOT) and its V into registers.
template <bool OUT, int W, bool SLOT = true>
__device__ __forceinline__ void scan_issue(ScanBuf<OUT>* buf, const ScanCtx& cx, int c,
                                           u32x2 (&vf)[4]) {
  const int wave = wave_index(), lane = threadIdx.x & 63;
  const int tc = cx.start + c * kChunk;
  const int nc = min(kChunk, cx.end - tc);
  scan_dma<OUT, W, SLOT>(*buf, cx.k + (static_cast<size_t>(tc) * cx.H + cx.h) * kDim,
                   cx.q + (static_cast<size_t>(tc) * cx.H + cx.h) * kDim, cx.kstep, nc,
                   cx.slot_base + c * cx.slot_step, wave, lane);
  load_v(vf, cx.v + (static_cast<size_t>(tc) * cx.HV + cx.hv) * kDim, cx.vstep, nc,
         column_wave<W>(cx, wave), lane & 15, lane >> 4);
}

// Where chunk c's inputs come from (rows >= n repeat row n - 1).
struct ChunkSrc {
  const uint16_t* kbase;
  const uint16_t* qbase;
  const uint16_t* vbase;
  const float* slot;
  int n;
};

__device__ __forceinline__ ChunkSrc chunk_src(const ScanCtx& cx, int c) {
  const int tc = cx.start + c * kChunk;
  ChunkSrc s;
  s.kbase = cx.k + (static_cast<size_t>(tc) * cx.H + cx.h) * kDim;
  s.qbase = cx.q + (static_cast<size_t>(tc) * cx.H + cx.h) * kDim;
  s.vbase = cx.v + (static_cast<size_t>(tc) * cx.HV + cx.hv) * kDim;
  s.slot = cx.slot_base + c * cx.slot_step;
  s.n = min(kChunk, cx.end - tc);
  return s;
}

// Part `part` (0..3) of a chunk's DMA and V loads, so that a chunk step
// spreads them over its products (issued at once, the eight waves' DMA
// instructions queue behind each other and hold each wave at the issue for
// 1-2.5 k cycles): with W = 8, parts 0..2 the K / Q row instructions w + 8
// part, part 2 also slot instruction w, part 3 slot instruction w + 8 and the
// V loads; with W = 4 each part issues twice as many, instructions w + 4 j
// for j = 2 part, 2 part + 1 (rows) and j = 2 (part - 2), 2 (part - 2) + 1
// (slot).
template <bool OUT, int W>
__device__ __forceinline__ void issue_part(ScanBuf<OUT>* __restrict__ Bn, const ScanCtx& cx,
                                           const ChunkSrc& s, int part, u32x2 (&vf)[4]) {
  constexpr int kPer = kScanWaves / W;                      // instructions a wave a part
  const int wave = wave_index(), lane = threadIdx.x & 63;
  if (part < 3) {
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int i = wave + W * (kPer * part + j);
      if (i < kRowDma) {                                    // uniform per wave
        const int pc = i * 64 + lane;
        const int r = pc / kRowPieces, c = pc % kRowPieces;
        const unsigned off = row_bytes(r < s.n ? r : s.n - 1, cx.kstep, (c < 16 ? c : 15) * 8);
        dma16_at(s.kbase, off, &Bn->Kr[i * 512]);
        if constexpr (OUT) dma16_at(s.qbase, off, &Bn->Qr[i * 512]);
      }
    }
  }
  if (part >= 2) {
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int i = wave + W * (kPer * (part - 2) + j);
      if (i < kSlotDma)
        dma16_at(s.slot, static_cast<unsigned>(i * 64 + lane) * 16u, &Bn->slot[i * 256]);
    }
  }
  if (part == 3)
    load_v(vf, s.vbase, cx.vstep, s.n, column_wave<W>(cx, wave), lane & 15, lane >> 4);
}

// P' tiles (row tile r, token tile jt) of a chunk, 10 nonzero and the two
// zero ones inside the stored blocks (0, 1) and (2, 3); wave w of W makes
// tiles w, w + W, ....
// Tile idx is (r, jt) = ((kPTileR >> 2 idx) & 3, (kPTileJ >> 2 idx) & 3):
//   r  = 0, 1, 1, 2, 2, 2, 3, 3, 3, 3, 0, 2
//   jt = 0, 0, 1, 0, 1, 2, 0, 1, 2, 3, 1, 3
// (packed in immediates: a table in memory costs a global load and its wait
// at the start of every chunk step).
constexpr int kPTiles = 12;
constexpr unsigned kPTileR = 0x8ffa94u;
constexpr unsigned kPTileJ = 0xde4910u;

// Key block kb's product of P' tile IDX, (K Q^T)_(jt, r) over the block,
// from the K and Q operands of the block's row tiles (in registers).
template <int IDX>
__device__ __forceinline__ void p_tile_mma(const s16x8 (&ak)[4], const s16x8 (&bq)[4],
                                           f32x4& acc) {
  constexpr int r = (kPTileR >> (2 * IDX)) & 3, jt = (kPTileJ >> (2 * IDX)) & 3;
  if constexpr (jt <= r) acc = mfma_bf16(ak[jt], bq[r], acc);
}

// Chunk ci from buffer B, with the next chunk's DMA into Bn; Kt: the K^T
// operand blocks; Pb: the P' operand blocks (OUT); Qn: the Q row scales
// (L2).  B, Bn, Kt, Pb and Qn are restrict: the compiler then knows that the
// DMA in flight into Bn never writes what this chunk reads, and waits for it
// only at the end.  OUT: the outputs too (else only the state).  L2: the
// L2-norm (a template flag: as a run-time branch inside the product loop it
// split the loop into blocks the scheduler could not interleave).
//
// The output's intra-chunk term uses P = diag(rq) P' with
//   P'_ij = scale rk_j e^(gamma_i - gamma_j) (Q K^T)_ij,  j <= i,
// made here from the chunk's K and Q rows: (K Q^T) tiles on bf16 MFMA leave
// each lane 4 consecutive j of one row i, the operand items of P' as the B
// operand of Delta^T P'^T.  The Q row scales rq = 1 / |q_i| (L2-norm; each
// wave computes eight rows' from the Q rows in LDS and shares them through
// Qn) scale the output row: O = diag(rq) (diag(scale e^gamma) Q S + P' Delta).
template <bool OUT, bool L2, int W, bool FUSE = false>
__device__ __forceinline__ void scan_chunk(const ScanBuf<OUT>* __restrict__ B,
                                           ScanBuf<OUT>* __restrict__ Bn,
                                           uint16_t* __restrict__ Kt, uint16_t* __restrict__ Pb,
                                           float* __restrict__ Qn, const ScanCtx& cx,
                                           f32x4 (&st)[8],
                                           u32x2 (&vnext)[4], const s16x8& sel, int ci) {
  const int lane = threadIdx.x & 63;
  const int wave = wave_index();
  const int col = lane & 15;
  const int g4 = lane >> 4;
  const int t0 = cx.start + ci * kChunk;
  const int n = min(kChunk, cx.end - t0);
  const int cw = column_wave<W>(cx, wave);   // columns 16 cw .. 16 cw + 15
  const u32x2 vf[4] = {vnext[0], vnext[1], vnext[2], vnext[3]};
  // The next chunk's inputs go into the other buffer (after the last chunk:
  // this one's again, unused) in four parts spread over the K S products.
  const ChunkSrc nsrc = chunk_src(cx, ci + 1 < cx.nchunks ? ci + 1 : ci);
  // The chunk's row scales are read where they are used, so that they hold
  // no registers across the products: B is restrict and 16-byte aligned, so
  // each read is one ds_read_b128 that the compiler knows the DMA in flight
  // into Bn does not write (reads it splits into pairs of 4-byte reads lose
  // that, and wait for the DMA).

  // L2-norm: 1 / |q_i| of Q rows 8 v .. 8 v + 7 into Qn, v = wave + W rep
  // (lane: row 8 v + lane / 8, items 16 (lane % 8) .. + 15); read after the
  // barrier below.  (The previous chunk's reads of Qn ended before its last
  // barrier.)
  if constexpr (L2) {
#pragma unroll
    for (int rep = 0; rep < kScanWaves / W; ++rep) {
      const int row = 8 * (wave + W * rep) + (lane >> 3);
      const uint16_t* qr = &B->Qr[row * kRowStride + (lane & 7) * 16];
      const u32x4 w[2] = {*reinterpret_cast<const u32x4*>(qr),
                          *reinterpret_cast<const u32x4*>(qr + 8)};
      float q2 = 0.0f;
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float lo = __uint_as_float(w[h][i] << 16);
          const float hi = __uint_as_float(w[h][i] & 0xffff0000u);
          q2 = fmaf(hi, hi, fmaf(lo, lo, q2));
        }
      q2 += __shfl_xor(q2, 1, 64);
      q2 += __shfl_xor(q2, 2, 64);
      q2 += __shfl_xor(q2, 4, 64);
      if ((lane & 7) == 0) Qn[row] = __builtin_amdgcn_rsqf(q2 + kL2Eps);
    }
  }

  // K S (token rows) and S^T Q^T (the output's first term, transposed),
  // one 32-key block of the state at a time.  The K and Q operands of key
  // block kb + 1 are read into the other of two register sets while block
  // kb's products run, so the LDS latency is paid once, not per product.
  // The same operands make this wave's key tiles of K^T (tiles t = wave +
  // W m, key block t / 2: the selector products of the K row tiles give lane
  // (col, g) tokens 16 r + 4 g + e of key state_key(t, col / 4) + col % 4)
  // and its P' tiles' (K Q^T) products, shared with the other waves through
  // LDS.
  constexpr int kKtTiles = kScanWaves / W;                  // K^T tiles a wave makes
  constexpr int kPReps = (kPTiles + W - 1) / W;             // P' tiles a wave makes, at most
  f32x4 x[4], o[4], pacc[kPReps];
#pragma unroll
  for (int r = 0; r < 4; ++r) x[r] = o[r] = f32x4{0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < kPReps; ++i) pacc[i] = f32x4{0, 0, 0, 0};
  s16x4 kt[kKtTiles][4];
  s16x8 ak[2][4], bq[2][4];
  auto read_ops = [&](int kb, int set) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      ak[set][r] = frag(&B->Kr[(r * 16 + col) * kRowStride], kb, g4);
      if constexpr (OUT) bq[set][r] = frag(&B->Qr[(r * 16 + col) * kRowStride], kb, g4);
    }
  };
  read_ops(0, 0);
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    const int set = kb & 1;
    if (kb < 3) read_ops(kb + 1, set ^ 1);
    if constexpr (!FUSE) issue_part<OUT, W>(Bn, cx, nsrc, kb, vnext);   // FUSE: one chunk
#pragma unroll
    for (int m = 0; m < kKtTiles; ++m) {
      if (kb == ((wave + W * m) >> 1)) {                    // uniform per wave
#pragma unroll
        for (int r = 0; r < 4; ++r)
          kt[m][r] = to_bf16x4(mfma_bf16(ak[set][r], sel, f32x4{0, 0, 0, 0}));
      }
    }
    if constexpr (OUT && W == 8) {
      switch (wave) {                                       // uniform per wave
        case 0: p_tile_mma<0>(ak[set], bq[set], pacc[0]); p_tile_mma<8>(ak[set], bq[set], pacc[1]); break;
        case 1: p_tile_mma<1>(ak[set], bq[set], pacc[0]); p_tile_mma<9>(ak[set], bq[set], pacc[1]); break;
        case 2: p_tile_mma<2>(ak[set], bq[set], pacc[0]); break;
        case 3: p_tile_mma<3>(ak[set], bq[set], pacc[0]); break;
        case 4: p_tile_mma<4>(ak[set], bq[set], pacc[0]); break;
        case 5: p_tile_mma<5>(ak[set], bq[set], pacc[0]); break;
        case 6: p_tile_mma<6>(ak[set], bq[set], pacc[0]); break;
        default: p_tile_mma<7>(ak[set], bq[set], pacc[0]); break;
      }
    } else if constexpr (OUT) {                             // W = 4: tiles w, w + 4, w + 8
      switch (wave) {                                       // uniform per wave
        case 0: p_tile_mma<0>(ak[set], bq[set], pacc[0]); p_tile_mma<4>(ak[set], bq[set], pacc[1]);
                p_tile_mma<8>(ak[set], bq[set], pacc[2]); break;
        case 1: p_tile_mma<1>(ak[set], bq[set], pacc[0]); p_tile_mma<5>(ak[set], bq[set], pacc[1]);
                p_tile_mma<9>(ak[set], bq[set], pacc[2]); break;
        case 2: p_tile_mma<2>(ak[set], bq[set], pacc[0]); p_tile_mma<6>(ak[set], bq[set], pacc[1]);
                p_tile_mma<10>(ak[set], bq[set], pacc[2]); break;
        default: p_tile_mma<3>(ak[set], bq[set], pacc[0]); p_tile_mma<7>(ak[set], bq[set], pacc[1]);
                 p_tile_mma<11>(ak[set], bq[set], pacc[2]); break;
      }
    }
    s16x8 sl;
    const s16x8 sh = split_hi_lo(st[2 * kb], st[2 * kb + 1], sl);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      x[r] = mfma_bf16(ak[set][r], sh, x[r]);
      if constexpr (OUT) o[r] = mfma_bf16(sh, bq[set][r], o[r]);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      x[r] = mfma_bf16(ak[set][r], sl, x[r]);
      if constexpr (OUT) o[r] = mfma_bf16(sl, bq[set][r], o[r]);
    }
  }

  // this wave's K^T tiles and P' tiles into LDS (read after the barrier below)
#pragma unroll
  for (int m = 0; m < kKtTiles; ++m)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
      *reinterpret_cast<s16x8*>(Kt + (((wave + W * m) * 2 + kb) * 64 + lane) * 8) =
          cat(kt[m][2 * kb], kt[m][2 * kb + 1]);
  if constexpr (OUT) {
    // P' tile (r, jt): lane (col, g) holds row i = 16 r + col, tokens
    // j = 16 jt + 4 g + e; items 4 (jt % 2) .. + 3 of block (r, jt / 2)
#pragma unroll
    for (int rep = 0; rep < kPReps; ++rep) {
      const int idx = wave + W * rep;
      if (idx >= kPTiles) break;                       // uniform per wave
      const int r = (kPTileR >> (2 * idx)) & 3, jt = (kPTileJ >> (2 * idx)) & 3;
      f32x4 pv = {0, 0, 0, 0};
      if (jt <= r) {                                   // uniform per wave
        const int i = r * 16 + col, j0 = jt * 16 + g4 * 4;
        const float gi = B->slot[kSlotGa + i];
        const f32x4 gj = *reinterpret_cast<const f32x4*>(&B->slot[kSlotGa + j0]);
        const f32x4 rkj = *reinterpret_cast<const f32x4*>(&B->slot[kSlotRk + j0]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x = cx.scale * rkj[e] * __expf(fminf(gi - gj[e], 0.0f)) * pacc[rep][e];
          pv[e] = j0 + e <= i ? x : 0.0f;
        }
      }
      s16x4 hi, lo;
      split4(pv, hi, lo);
      const int at = tri_blk(r, jt >> 1) * kBlk + lane * 8 + (jt & 1) * 4;
      *reinterpret_cast<s16x4*>(Pb + at) = hi;
      *reinterpret_cast<s16x4*>(Pb + kTriBlocks * kBlk + at) = lo;
    }
  }

  // T diag(beta)'s six lower operand blocks (hi, lo), read while X is formed
  s16x8 th[kTriBlocks], tl[kTriBlocks];
#pragma unroll
  for (int b = 0; b < kTriBlocks; ++b) {
    th[b] = ld_op(&B->slot[kSlotTh + b * kBlkF + lane * 4]);
    tl[b] = ld_op(&B->slot[kSlotTl + b * kBlkF + lane * 4]);
  }

  // X = V - diag(rk e^gamma) K S: lane (col, g) holds tokens 16 r + 4 g + e
  // of column 16 cw + col; V^T tiles from the selector products (the
  // wave's 16 columns sit in the half `cw % 2` = `wave % 2` of a 32-column
  // block)
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const f32x4 xg = *reinterpret_cast<const f32x4*>(&B->slot[kSlotXg + r * 16 + g4 * 4]);
    const u32x2 vv = cx.values ? vf[r] : u32x2{0u, 0u};
    const u32x4 w4 = (wave & 1) ? u32x4{0u, 0u, vv.x, vv.y} : u32x4{vv.x, vv.y, 0u, 0u};
    const f32x4 v = mfma_bf16(__builtin_bit_cast(s16x8, w4), sel, f32x4{0, 0, 0, 0});
    x[r] = v - xg * x[r];
  }

  // Delta = T diag(beta) X (T lower triangular: token blocks kb <= r / 2)
  s16x8 xh[2], xl[2];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) xh[kb] = split_hi_lo(x[2 * kb], x[2 * kb + 1], xl[kb]);
  f32x4 d[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    d[r] = f32x4{0, 0, 0, 0};
#pragma unroll
    for (int kb = 0; kb <= (r >> 1); ++kb) {
      const int b = tri_blk(r, kb);
      d[r] = mfma_bf16(th[b], xh[kb], d[r]);
      d[r] = mfma_bf16(th[b], xl[kb], d[r]);
      d[r] = mfma_bf16(tl[b], xh[kb], d[r]);
    }
  }

  // Delta as operand: A of Delta^T P^T and, scaled by ks, B of the update
  s16x8 dh[2], dl[2], eh[2], el[2];
  f32x4 ks[4];
#pragma unroll
  for (int r = 0; r < 4; ++r)
    ks[r] = *reinterpret_cast<const f32x4*>(&B->slot[kSlotKs + r * 16 + g4 * 4]);
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    if constexpr (OUT) dh[kb] = split_hi_lo(d[2 * kb], d[2 * kb + 1], dl[kb]);
    eh[kb] = split_hi_lo(d[2 * kb] * ks[2 * kb], d[2 * kb + 1] * ks[2 * kb + 1], el[kb]);
  }

  // every wave's K^T tile and P' tiles are in LDS past this barrier
  barrier_lds_no_dma();

  // The operands of the output products two row tiles ahead of their use,
  // and those of the state update in two halves, the first read with the
  // output's, the second while the first half's products run.
  s16x8 ph[kTriBlocks], pl[kTriBlocks], kt_op[8][2];
  auto read_p = [&](int r) {
#pragma unroll
    for (int kb = 0; kb <= (r >> 1); ++kb) {
      const int b = tri_blk(r, kb);
      ph[b] = ld_op(Pb + b * kBlk + lane * 8);
      pl[b] = ld_op(Pb + (kTriBlocks + b) * kBlk + lane * 8);
    }
  };
  if constexpr (OUT) {
    read_p(0);
    read_p(1);
  }
  auto read_kt = [&](int t0k) {
#pragma unroll
    for (int t = t0k; t < t0k + 4; ++t)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) kt_op[t][kb] = ld_op(Kt + ((t * 2 + kb) * 64 + lane) * 8);
  };
  read_kt(0);

  // O^T = rq (.) (qs (.) S^T Q^T + Delta^T P'^T); lane (col, g) ends with
  // columns 16 cw + 4 g + e of token 16 r + col, one 8-byte store
  if constexpr (OUT) {
    uint16_t* const obase = cx.out + (static_cast<size_t>(t0) * cx.HV + cx.hv) * kDim;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (r < 2) read_p(r + 2);
      o[r] = o[r] * (cx.scale * B->slot[kSlotEg + r * 16 + col]);
#pragma unroll
      for (int kb = 0; kb <= (r >> 1); ++kb) {
        const int b = tri_blk(r, kb);
        o[r] = mfma_bf16(dh[kb], ph[b], o[r]);
        o[r] = mfma_bf16(dh[kb], pl[b], o[r]);
        o[r] = mfma_bf16(dl[kb], ph[b], o[r]);
      }
      if constexpr (L2) o[r] = o[r] * Qn[r * 16 + col];
      const int tok = r * 16 + col;
      const u32x2 ob = {pack_bf16x2(o[r][0], o[r][1]), pack_bf16x2(o[r][2], o[r][3])};
      if (tok < n)
        *reinterpret_cast<u32x2*>(reinterpret_cast<char*>(obase) +
                                  row_bytes(tok, cx.vstep, cw * 16 + g4 * 4)) = ob;
    }
  }

  // S <- e^gamma_C S + K^T (ks (.) Delta), key tile t
  const float gl = B->slot[kSlotGl];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    if (t == 1) read_kt(4);
    f32x4 acc = st[t] * gl;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      acc = mfma_bf16(kt_op[t][kb], eh[kb], acc);
      acc = mfma_bf16(kt_op[t][kb], el[kb], acc);
    }
    st[t] = acc;
  }

  wait_vmem();                       // the next chunk's DMA has landed
  block_sync_lds();                  // for every wave; this chunk's LDS reads are done
}

// The end state of a scan: k-last fp32 (element (k, c) at c * 128 + k), or,
// for a transition M (identity start), as the A operand blocks of the
// combine's product M S: for row tile t and column block kb, 64 lanes x 8
// bf16, hi then lo (block ((t * 4 + kb) * 2 + hl) * 512).  Column wave w
// (cw: the wave's columns 16 w .. 16 w + 15) is half w % 2 of block kb = w /
// 2: the selector products of its state read as an operand with the columns
// as rows give lane (col, g) the columns 16 w + 4 g + e of row state_key(t,
// col / 4) + col % 4, items 4 (w % 2) .. + 3 of the block's lane; those
// columns started from start keys 32 kb + 8 g + item, the key order of the
// combine's S operand.
__device__ __forceinline__ void store_end(float* st_out, bool transition, const f32x4 (&st)[8],
                                          const s16x8 (&sels)[2], int cw) {
  const int lane = threadIdx.x & 63;
  const int wave = cw;
  const int col = lane & 15;
  const int g4 = lane >> 4;
  if (!transition) {
#pragma unroll
    for (int t = 0; t < 8; ++t)
      *reinterpret_cast<f32x4*>(st_out + static_cast<size_t>(wave * 16 + col) * kDim +
                                state_key(t, g4)) = st[t];
    return;
  }
  uint16_t* ma = reinterpret_cast<uint16_t*>(st_out);
#pragma unroll
  for (int kb2 = 0; kb2 < 4; ++kb2) {                 // rows 32 kb2 .. 32 kb2 + 31
    s16x8 al;
    const s16x8 ah = split_hi_lo(st[2 * kb2], st[2 * kb2 + 1], al);
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int t = 2 * kb2 + hf;
      const int blk0 = (t * 4 + (wave >> 1)) * 2;
      const int item = lane * 8 + (wave & 1) * 4;
      *reinterpret_cast<s16x4*>(ma + blk0 * kBlk + item) =
          to_bf16x4(mfma_bf16(ah, sels[hf], f32x4{0, 0, 0, 0}));
      *reinterpret_cast<s16x4*>(ma + (blk0 + 1) * kBlk + item) =
          to_bf16x4(mfma_bf16(al, sels[hf], f32x4{0, 0, 0, 0}));
    }
  }
}

// Grid: (unit, q/k head) pairs in groups of 8 times the GVA ratio times the
// column halves (W = 4: 2, W = 8: 1).  Workgroup b serves pair 8 (b / (8
// ratio halves)) + b % 8 and, with m = (b / 8) % (ratio halves), its v-head
// m % ratio and half m / ratio: the workgroups that read the same K and Q
// are dispatched 8 apart, all to XCD b % 8 (workgroups go to the XCDs
// round-robin), and share its L2 copy.  A unit is a sequence, or with SEG a role of one segment of
// sequence 0.  The first segment launch (OUT false, no outputs) runs
// segment 0 from the sequence's state (end: seg_S[1]) and segments
// 1 .. nseg-2 from a zero start (end: seg_B) and from the identity without
// values (end: seg_M, as the combine's operand); the second (OUT) runs every
// segment from its start (segment 0: the sequence's state, then seg_S) with
// the outputs, the last one's end being the new state.
template <bool FEW, bool SEG, bool OUT, bool L2, int W, bool FUSE>
__device__ __forceinline__ void scan_body(Params p) {
  static_assert(OUT || SEG, "only segments run without outputs");
  static_assert(!FUSE || (!FEW && !SEG && OUT && W == kThreads / 64),
                "the one-chunk kernel: half-state workgroups of the preparation's width");
  static_assert(OUT || !L2, "the L2-norm scales outputs only");
  static_assert(W == kScanWaves || (W == kScanWaves / 2 && !SEG),
                "half-state workgroups run plain scans only");
  constexpr int kHalves = kScanWaves / W;
  // separate LDS objects, so that the compiler sees that the DMA into one
  // buffer never writes what the chunk reads from the other
  __shared__ ScanBuf<OUT> L0, L1;
  __shared__ __attribute__((aligned(16))) uint16_t Kt[kKtElems];
  __shared__ __attribute__((aligned(16))) uint16_t Pb[OUT ? kPElems : 8];
  __shared__ float Qn[L2 ? kChunk : 1];    // 1 / |q_i| of the chunk's Q rows (L2-norm)
  const long long b = blockIdx.x;
  const int ratio = p.ratio;
  const long long pair = (b / (8LL * ratio * kHalves)) * 8 + (b & 7);
  const int member = static_cast<int>((b >> 3) % (ratio * kHalves));
  const int jr = member % ratio;
  const int cw0 = W == kScanWaves ? 0 : (member / ratio) * W;   // the first wave's column wave
  // units the grid covers: with SEG the launch's bound, each workgroup
  // finding its sequence's segment below (those past the batch's exit)
  const long long units = SEG ? (OUT ? p.nseg : seg_units1(p.nseg, p.N))
                              : static_cast<long long>(p.N);
  if (pair >= units * p.H) return;                              // uniform per workgroup
  if (p.short_limit > 0 && all_within(p, p.short_limit)) return;  // uniform
  const int unit = static_cast<int>(pair / p.H);
  const int h = static_cast<int>(pair % p.H);
  const int hv = h * ratio + jr;
  const int lane = threadIdx.x & 63;
  const int wave = wave_index();
  const int col = lane & 15;
  const int g4 = lane >> 4;
  const size_t blk = static_cast<size_t>(kDim) * kDim;

  // role: start state, values, where the end state goes
  const float* st_in = nullptr;       // null: zeros (or the identity)
  bool identity = false, values = true, pass_through = false;
  float* st_out;
  int s = 0, start, end, slot0 = 0, nchunks = 0;
  // the sequence's chunk slots (never more than its range holds, and never
  // more slots than the workspace has, whatever cu_seqlens contains)
  auto seq_slots = [&](int sq, int& base, int& count) {
    if (p.single) {
      base = 0;
      count = (end - start + kChunk - 1) / kChunk;
    } else if (FEW) {
      const FewSlots f = few_slots(p);
      base = static_cast<int>(__shfl(f.excl, sq, 64));
      count = static_cast<int>(__shfl(f.incl, sq, 64)) - base;
    } else {
      base = p.offs[sq];
      count = p.offs[sq + 1] - base;
    }
  };
  if (SEG) {
    const SegSeqs f = seg_seqs<OUT>(p);
    const unsigned long long own = __ballot(lane < p.N && f.u_excl <= unit && unit < f.u_incl);
    if (own == 0) return;                         // past the batch's units (uniform)
    s = __builtin_ctzll(own);                     // uniform: lane reads, no shuffles
    const int nseg = __builtin_amdgcn_readlane(f.nseg, s);
    const int g0 = __builtin_amdgcn_readlane(f.seg_excl, s);   // the sequence's first segment
    if (g0 + nseg > p.nseg) return;               // past the workspace's (a malformed batch)
    const int u = unit - __builtin_amdgcn_readlane(f.u_excl, s);
    start = __builtin_amdgcn_readlane(f.start, s);
    end = __builtin_amdgcn_readlane(f.end, s);
    const size_t sh = static_cast<size_t>(s) * p.HV + hv;        // the sequence's state
    auto seg_blk = [&](float* base, int g) { return base + (static_cast<size_t>(g) * p.HV + hv) * blk; };
    int j;
    if (!OUT) {
      const int mid = nseg - 2;                   // segments 1 .. nseg-2
      if (u == 0) {
        j = 0;
        st_in = p.state ? p.state + sh * blk : nullptr;
        st_out = seg_blk(p.seg_S, g0 + 1);
      } else if (u <= mid) {
        j = u;
        st_out = seg_blk(p.seg_B, g0 + j);
      } else {
        j = u - mid;
        identity = true;
        values = false;
        st_out = seg_blk(p.seg_M, g0 + j);
      }
    } else {
      j = u;
      st_in = j == 0 ? (p.state ? p.state + sh * blk : nullptr) : seg_blk(p.seg_S, g0 + j);
      st_out = j == nseg - 1 ? p.new_state + sh * blk : nullptr;
      pass_through = j > 0;
    }
    int base, count;
    seq_slots(s, base, count);
    const int first = j * p.seg_chunks;
    slot0 = base + first;
    // the last segment takes the rest (at most seg_chunks, but the whole
    // sequence when a malformed batch runs every sequence as one segment)
    nchunks = j == nseg - 1 ? count - first : min(p.seg_chunks, count - first);
    start = min(end, start + first * kChunk);
    if (nchunks > 0) end = min(end, start + nchunks * kChunk);
  } else {
    s = unit;
    seq_range(p, s, start, end);
    st_in = p.state ? p.state + (static_cast<size_t>(s) * p.HV + hv) * blk : nullptr;
    st_out = p.new_state + (static_cast<size_t>(s) * p.HV + hv) * blk;
    if constexpr (FUSE)
      nchunks = end > start ? 1 : 0;    // every sequence is one chunk (at most 64 tokens in all)
    else
      seq_slots(s, slot0, nchunks);
  }

  // state registers (keys in the order of state_key); k-last storage: 4
  // consecutive keys are one 16-byte vector.  The identity start of a
  // transition gives column 16 w + m the unit vector of the key in register
  // position (w, m): key state_key(w, m / 4) + m % 4, so that its end column
  // is that start key's column of M, in the key order of the combine's
  // operand.  (w: the column wave, cw0 + wave.)
  f32x4 st[8];
  const int cw = cw0 + wave;
  const int c = cw * 16 + col;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    st[t] = st_in != nullptr && (end > start || pass_through)
                ? *reinterpret_cast<const f32x4*>(st_in + static_cast<size_t>(c) * kDim +
                                                  state_key(t, g4))
                : f32x4{0, 0, 0, 0};
    if (identity) {
#pragma unroll
      for (int e = 0; e < 4; ++e) st[t][e] = t == cw && 4 * g4 + e == col ? 1.0f : 0.0f;
    }
  }
  // selector operands: Sel_h[k][j] = (k == 16 h + j) over a 32-long k block
  s16x8 sels[2];
#pragma unroll
  for (int hf = 0; hf < 2; ++hf)
#pragma unroll
    for (int e = 0; e < 8; ++e)
      sels[hf][e] = (e == 4 * hf + (col & 3) && g4 == (col >> 2)) ? 0x3f80 : 0;

  // No tokens: a sequence ends in zeros, as the reference; a segment with no
  // chunk slots (a malformed batch whose slots ran past the workspace's)
  // passes its start through (transition: the identity, zero-start end:
  // zeros), and so does the sequence's end state.
  if (nchunks <= 0) {
    if (st_out != nullptr) {
      if (!SEG) {
#pragma unroll
        for (int t = 0; t < 8; ++t) st[t] = f32x4{0, 0, 0, 0};
      }
      store_end(st_out, identity, st, sels, cw);
    }
    return;
  }
  ScanCtx cx;
  cx.k = p.k;
  cx.q = p.q;
  cx.v = p.v;
  cx.out = p.out;
  cx.slot_base = p.slots + (static_cast<size_t>(slot0) * p.HV + hv) * kSlotFloats;
  cx.slot_step = static_cast<size_t>(p.HV) * kSlotFloats;
  cx.kstep = static_cast<unsigned>(p.H) * kDim;
  cx.vstep = static_cast<unsigned>(p.HV) * kDim;
  cx.start = start;
  cx.end = end;
  cx.nchunks = nchunks;
  cx.H = p.H;
  cx.HV = p.HV;
  cx.h = h;
  cx.hv = hv;
  cx.values = values;
  cx.scale = p.scale;
  cx.cw0 = cw0;

  const s16x8 sel = sels[wave & 1];       // this wave's half of a 32-key / 32-column block
  u32x2 vnext[4];
  if constexpr (FUSE) {
    // The chunk's K and Q rows by DMA and its V while this workgroup prepares
    // its slot in LDS (the preparation's LDS in the second buffer, which one
    // chunk never uses), then its one chunk step.
    static_assert(sizeof(PrepLds) <= sizeof(ScanBuf<OUT>), "the preparation fits a buffer");
    scan_issue<OUT, W, false>(&L0, cx, 0, vnext);
    prep_chunk<true>(p, 0, start, end - start, hv, h, 1, *reinterpret_cast<PrepLds*>(&L1),
                     L0.slot);
    wait_vmem();
    block_sync_lds();
    scan_chunk<OUT, L2, W, true>(&L0, &L1, Kt, Pb, Qn, cx, st, vnext, sel, 0);
    if (st_out != nullptr) store_end(st_out, identity, st, sels, cw);
    return;
  }
  scan_issue<OUT, W>(&L0, cx, 0, vnext);
  wait_vmem();
  block_sync_lds();
  for (int ci = 0; ci < nchunks; ci += 2) {
    scan_chunk<OUT, L2, W>(&L0, &L1, Kt, Pb, Qn, cx, st, vnext, sel, ci);
    if (ci + 1 < nchunks)                                                      // uniform
      scan_chunk<OUT, L2, W>(&L1, &L0, Kt, Pb, Qn, cx, st, vnext, sel, ci + 1);
  }
  if (st_out != nullptr) store_end(st_out, identity, st, sels, cw);
}

template <bool FEW, bool SEG, bool OUT, bool L2, int W>
__global__ __launch_bounds__(64 * W)
__attribute__((amdgpu_waves_per_eu(W == kScanWaves ? 2 : 1, W == kScanWaves ? 2 : 1)))
void scan_kernel(Params p) {
  scan_body<FEW, SEG, OUT, L2, W, false>(p);
}

// Prefills whose tokens all fit one chunk: each (sequence, v-head, half)
// workgroup prepares its sequence's chunk in LDS and scans it, in one launch.
template <bool L2>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void one_chunk_kernel(Params p) {
  scan_body<false, false, true, L2, kThreads / 64, true>(p);
}

// ---------------------------------------------------------------------------
// 4. segments: chain each sequence's segment starts
// ---------------------------------------------------------------------------
// The first segment launch leaves, per (sequence, v-head), S_1 and for each
// middle segment j its transition M_j (as the A operand blocks of M S, bf16
// hi/lo) and zero-start end B_j.  Combine: S_{j+1} = M_j S_j + B_j for j = 1
// .. nseg-2, segment after segment, as bf16 MFMA with S_j split into hi + lo.
// One workgroup per (sequence, v-head, 16 state columns); wave w computes row
// tile w (in the scan's key order: rows state_key(w, i / 4) + i % 4, the rows
// of M's tile w) and hands its rows of S_j to the other waves as half of the
// B operand's k block w / 2 through LDS (two buffers: one barrier a step).  A step is short (12 MFMAs a wave), so each wave's M
// blocks and B tile are loaded three steps ahead, into three register sets
// used in turn.  Every workgroup reads all of M_j: the eight of a (sequence,
// v-head) are numbered hv + 8k within the sequence's (HV rounded up to 8
// between them), so all of them run on XCD hv % 8 (workgroups go to the XCDs
// round-robin) and read M_j from its L2 after the first.
constexpr int kCombWaves = 8;

struct CombStage {
  s16x8 ma[4][2];                             // [k block][hi, lo] of row tile w
  f32x4 bt;                                   // B_j rows of row tile w
};

__global__ __launch_bounds__(64 * kCombWaves) void seg_combine_kernel(Params p) {
  __shared__ s16x8 Sop[2][4][2][64];          // [buffer][k block][hi, lo][lane]
  const int hv_pad = (p.HV + 7) & ~7;
  const int per_seq = hv_pad * 8;
  const int sq = static_cast<int>(blockIdx.x) / per_seq;
  const int hv = static_cast<int>(blockIdx.x) % hv_pad;
  const int c0 = static_cast<int>(blockIdx.x) % per_seq / hv_pad * 16;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int col = lane & 15;
  const int g4 = lane >> 4;
  const size_t blk = static_cast<size_t>(kDim) * kDim;
  if (sq >= p.N || hv >= p.HV) return;        // padding (uniform)
  // the sequence's segments: one sequence has the workspace's (its chain
  // starts without reading cu_seqlens; steps past a shorter sequence's last
  // segment chain values nothing reads); several count theirs
  int nseg = p.nseg, g0 = 0;
  if (p.N > 1) {
    const SegSeqs f = seg_seqs<true>(p);
    nseg = __builtin_amdgcn_readlane(f.nseg, sq);
    g0 = __builtin_amdgcn_readlane(f.seg_excl, sq);
  }
  if (nseg < 3 || g0 + nseg > p.nseg) return; // nothing to chain; past the workspace's
  const int last = nseg - 2;                  // steps j = 1 .. last
  const size_t tile = static_cast<size_t>(c0 + col) * kDim + state_key(wave, g4);
  auto seg_blk = [&](const float* base, int j) {
    return base + (static_cast<size_t>(g0 + j) * p.HV + hv) * blk;
  };
  // S_1, this wave's row tile in the MFMA result layout
  f32x4 S = *reinterpret_cast<const f32x4*>(seg_blk(p.seg_S, 1) + tile);
  auto load = [&](int j, CombStage& cs) {     // past the last step: the last one's again
    j = j < last ? j : last;
    const uint16_t* M = reinterpret_cast<const uint16_t*>(seg_blk(p.seg_M, j));
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int hl = 0; hl < 2; ++hl)
        cs.ma[kb][hl] =
            *reinterpret_cast<const s16x8*>(M + (((wave * 4 + kb) * 2 + hl) * kBlk + lane * 8));
    cs.bt = *reinterpret_cast<const f32x4*>(seg_blk(p.seg_B, j) + tile);
  };
  auto step = [&](int j, CombStage& cs) {
    const int buf = j & 1;
    s16x4 hi, lo;
    split4(S, hi, lo);
    const int item = (wave & 1) * 4;
    uint16_t* sh16 = reinterpret_cast<uint16_t*>(&Sop[buf][wave >> 1][0][lane]);
    uint16_t* sl16 = reinterpret_cast<uint16_t*>(&Sop[buf][wave >> 1][1][lane]);
    *reinterpret_cast<s16x4*>(sh16 + item) = hi;
    *reinterpret_cast<s16x4*>(sl16 + item) = lo;
    block_sync_lds();
    f32x4 acc = cs.bt;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const s16x8 bh = Sop[buf][kb][0][lane];
      const s16x8 bl = Sop[buf][kb][1][lane];
      acc = mfma_bf16(cs.ma[kb][0], bh, acc);
      acc = mfma_bf16(cs.ma[kb][0], bl, acc);
      acc = mfma_bf16(cs.ma[kb][1], bh, acc);
    }
    S = acc;
    *reinterpret_cast<f32x4*>(const_cast<float*>(seg_blk(p.seg_S, j + 1)) + tile) = S;
    load(j + 3, cs);                          // this set's next use: three steps on
  };
  CombStage s0, s1, s2;
  load(1, s0);
  load(2, s1);
  load(3, s2);
  for (int j = 1; j <= last; j += 3) {        // uniform
    step(j, s0);
    if (j + 1 <= last) step(j + 1, s1);
    if (j + 2 <= last) step(j + 2, s2);
  }
}

bool aligned(const void* ptr, uintptr_t a) {
  return (reinterpret_cast<uintptr_t>(ptr) & (a - 1)) == 0;
}

size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

// Workspace: chunk offsets [N + 1] int32, slot table [max_slots] x 16 bytes,
// the v-head slots [max_slots, HV, kSlotFloats] fp32, then with segments
// their S, B and M blocks; each part 256-byte aligned.
size_t offsets_bytes(long long N) { return align256(static_cast<size_t>(N + 1) * sizeof(int32_t)); }

size_t slot_info_bytes(long long L, long long N) {
  return align256(static_cast<size_t>(max_slots(L, N)) * sizeof(i32x4));
}

size_t slots_bytes(long long L, long long N, long long HV) {
  return align256(static_cast<size_t>(max_slots(L, N)) * HV * kSlotFloats * sizeof(float));
}

// Segments.  A sequence's plain scan is a chain of chunk steps on HV
// workgroups; with few sequences and v-heads that leaves most of the GPU idle
// (16384 tokens at 8 v-heads: 256 steps on 8 CUs), so each sequence is cut
// into segments of len chunks scanned at once: the first launch runs 2 nseg
// - 3 units of a sequence of nseg segments (HV workgroups each), the second
// nseg, one workgroup per CU, each of len chunk steps, and the combine nseg -
// 2 small steps.  The host knows only the total tokens and the sequence
// count, so it plans for sequences of the mean length: the length is the one
// that minimises the estimated critical path, (rounds of the first launch +
// rounds of the second) x len chunk steps + (nseg - 2) combine steps + the
// two more launches, with a round of kCUs workgroups and a chunk step
// costing kStepPerCombine combine steps (measured: ~5.4 us against ~1 us);
// the batch is cut when that beats its plain scan, (rounds of N HV
// workgroups) x chunks x kStepPerCombine: from 6 chunks a sequence at N HV
// = 8 (one 2048-token sequence at qk4_v8: 195 -> ~66 us).  The kernels count
// each sequence's segments from cu_seqlens (so sequences shorter or longer
// than the mean get as many as they need), in one wave: at most kFewSeqs
// sequences.
constexpr long long kSegMaxHeads = 256;  // N HV workgroups that fill the GPU unsegmented
constexpr long long kSegMinLen = 2;
constexpr long long kCUs = 256;
constexpr long long kStepPerCombine = 5;
constexpr long long kSegLaunches = 8;    // the segment path's two more launches

struct SegPlan {
  long long len;    // chunks a segment (the mean sequence if not cut)
  long long cost;   // estimated critical path, combine steps; -1: cannot be cut
};

SegPlan seg_plan(long long L, long long N, long long HV) {
  const long long chunks = ((L + kChunk - 1) / kChunk + N - 1) / N;   // a sequence, mean
  SegPlan best{chunks, -1};
  for (long long len = kSegMinLen; 3 * len <= chunks; ++len) {
    const long long n = (chunks + len - 1) / len;
    const long long rounds =
        (N * (2 * n - 3) * HV + kCUs - 1) / kCUs + (N * n * HV + kCUs - 1) / kCUs;
    const long long cost = rounds * len * kStepPerCombine + (n - 2) + kSegLaunches;
    if (best.cost < 0 || cost < best.cost) best = SegPlan{len, cost};
  }
  return best;
}

// A plain scan whose whole-state workgroups (N HV) would fill at most half
// the CUs runs as half-state workgroups of 4 waves (two per (sequence,
// v-head), one wave a SIMD): chunk steps at about half the cost.
bool half_state_scan(long long N, long long HV) { return N >= 1 && 2 * N * HV <= kCUs; }

// Prefills past the token path whose tokens all fit one chunk (so every
// sequence is one chunk), with half-state workgroups that fit the GPU at
// once: one launch in which each (sequence, v-head, half) workgroup prepares
// its chunk in LDS and scans it -- no workspace round trip and one launch
// instead of the preparation's and the scan's.
bool fused_prefill(long long L, long long N, long long HV) {
  return L > kSmallTokens && L <= kChunk && half_state_scan(N, HV);
}

bool use_segments(long long L, long long N, long long HV) {
  if (N < 1 || N > kFewSeqs || N * HV > kSegMaxHeads) return false;
  const SegPlan plan = seg_plan(L, N, HV);
  const long long chunks = ((L + kChunk - 1) / kChunk + N - 1) / N;
  const long long whole = (N * HV + kCUs - 1) / kCUs * chunks * kStepPerCombine;
  return plan.cost >= 0 && plan.cost < whole;
}

long long seg_chunks(long long L, long long N, long long HV) { return seg_plan(L, N, HV).len; }

// Segments the workspace holds: one sequence's exactly; for several, the most
// a well-formed batch can have, sum(ceil(chunks_i / len)) <= (chunks + N
// (len - 1)) / len with chunks <= max_slots.  The kernels skip the segments of
// a (malformed) batch past this count.
long long num_segments(long long L, long long N, long long HV) {
  const long long len = seg_chunks(L, N, HV);
  if (N == 1) return ((L + kChunk - 1) / kChunk + len - 1) / len;
  return (max_slots(L, N) + N * (len - 1)) / len;
}

// Per segment and v-head one 128 x 128 fp32 block (S, B and M each).
size_t seg_blocks_bytes(long long L, long long N, long long HV) {
  return align256(static_cast<size_t>(num_segments(L, N, HV)) * HV * kDim * kDim * sizeof(float));
}

size_t workspace_bytes(long long L, long long N, long long H, long long HV) {
  (void)H;
  size_t bytes = offsets_bytes(N) + slot_info_bytes(L, N) + slots_bytes(L, N, HV);
  if (use_segments(L, N, HV)) bytes += 3 * seg_blocks_bytes(L, N, HV);
  return bytes;
}

}  // namespace gdn_pf

using namespace gdn_pf;

// One launch of the decode kernel's variable-length mode over the prefill's
// packed inputs: grid (row tiles x v-heads of a q/k head, q/k heads,
// sequences), one row per 16-lane group and one wave per workgroup for a few
// heads, four waves for more.
static hipError_t small_prefill(const void* q, const void* k, const void* v, const float* state,
                                const float* A_log, const void* a, const float* dt_bias,
                                const void* b, const int32_t* cu_seqlens, float scale,
                                void* output, float* new_state, int L, int N, int H, int HV,
                                bool l2, int short_limit, hipStream_t stream) {
  constexpr int kNs = 1;
  constexpr int kPolicy = gdn::kPolicyDefault;   // the next decode step re-reads the state
  const unsigned ratio = static_cast<unsigned>(HV / H);
  const unsigned h_ratio = static_cast<unsigned>(H) | (ratio << 16);
  const auto* q16 = static_cast<const uint16_t*>(q);
  const auto* k16 = static_cast<const uint16_t*>(k);
  const auto* v16 = static_cast<const uint16_t*>(v);
  const auto* a16 = static_cast<const uint16_t*>(a);
  const auto* b16 = static_cast<const uint16_t*>(b);
  auto* out16 = static_cast<uint16_t*>(output);
  if (static_cast<long long>(N) * HV <= 16) {
    constexpr int kW = 1;
    const dim3 grid(ratio * (kDim / (gdn::kLaneGroups * kNs * kW)), H, N);
    auto* kern = l2 ? gdn::gdn_decode_k128<kNs, kW, true, kPolicy, false, true, true>
                    : gdn::gdn_decode_k128<kNs, kW, false, kPolicy, false, true, true>;
    hipLaunchKernelGGL(kern, grid, dim3(64 * kW), 0, stream, state, q16, k16, v16, a16, b16,
                       h_ratio, 0, A_log, dt_bias, out16, new_state, scale, cu_seqlens, L,
                       short_limit);
  } else {
    constexpr int kW = 4;
    const dim3 grid(ratio * (kDim / (gdn::kLaneGroups * kNs * kW)), H, N);
    auto* kern = l2 ? gdn::gdn_decode_k128<kNs, kW, true, kPolicy, false, true, true>
                    : gdn::gdn_decode_k128<kNs, kW, false, kPolicy, false, true, true>;
    hipLaunchKernelGGL(kern, grid, dim3(64 * kW), 0, stream, state, q16, k16, v16, a16, b16,
                       h_ratio, 0, A_log, dt_bias, out16, new_state, scale, cu_seqlens, L,
                       short_limit);
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Fixed workspace of gdn_prefill_noalloc: a file-scope device array, so each
// GPU holds its own copy, at its own address, from the library's load on
// that GPU until the process ends.  Host code never passes the array's name
// to a kernel (on the host it is only a stand-in for the symbol): the
// device address comes from hipGetSymbolAddress, once per device, with that
// device current, and is cached per device.
// ---------------------------------------------------------------------------
constexpr size_t kScratchBytes = GDN_PREFILL_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
static std::atomic<void*> g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mutex;

// Device address of the current device's scratch array.
static hipError_t current_scratch(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  void* ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    ptr = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (ptr == nullptr) {
      e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return e;
      if (ptr == nullptr) return hipErrorInvalidSymbol;
      g_scratch_ptr[dev].store(ptr, std::memory_order_release);
    }
  }
  *out = ptr;
  return hipSuccess;
}

// fixed_scratch: the workspace is the current device's scratch array
// (workspace / workspace_size are ignored); sizes whose workspace exceeds it
// return hipErrorOutOfMemory before anything is launched.
static int prefill_impl(const void* q, const void* k, const void* v, const float* state,
                const float* A_log, const void* a, const float* dt_bias, const void* b,
                const int32_t* cu_seqlens, float scale, void* output, float* new_state,
                int total_seq_len, int num_seqs, int H, int HV, int K, int V,
                int use_qk_l2norm, void* workspace, size_t workspace_size,
                void* hip_stream, void* const* events, bool fixed_scratch = false) {
  if (total_seq_len < 0 || num_seqs < 0 || H <= 0 || HV <= 0 || HV % H != 0)
    return hipErrorInvalidValue;
  if (K != kDim || V != kDim) return hipErrorInvalidValue;
  if (HV > 65535) return hipErrorInvalidValue;      // grid y
  if (H > 32767) return hipErrorInvalidValue;       // packed in 15 bits for the token kernel
  if (num_seqs == 0) return hipSuccess;
  if (!cu_seqlens || !A_log || !dt_bias || !new_state || (!workspace && !fixed_scratch))
    return hipErrorInvalidValue;
  if (total_seq_len > 0 && (!q || !k || !v || !a || !b || !output))
    return hipErrorInvalidValue;
  const size_t need = workspace_bytes(total_seq_len, num_seqs, H, HV);
  if (fixed_scratch) {
    if (need > kScratchBytes) return hipErrorOutOfMemory;
    workspace = nullptr;                               // set once validation has passed
  } else if (workspace_size < need) {
    return hipErrorInvalidValue;
  }
  if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || !aligned(output, 16) ||
      !aligned(new_state, 16) || !aligned(state, 16) || !aligned(workspace, 256) ||
      !aligned(A_log, 4) || !aligned(dt_bias, 4) || !aligned(cu_seqlens, 4) ||
      !aligned(a, 2) || !aligned(b, 2))
    return hipErrorInvalidValue;
  if (state != nullptr && state == new_state) {
    // in place is fine: each scan workgroup reads its state slice before
    // writing it, and no two workgroups share a slice
  } else if (state != nullptr) {
    const uintptr_t s0 = reinterpret_cast<uintptr_t>(state);
    const uintptr_t d0 = reinterpret_cast<uintptr_t>(new_state);
    const size_t bytes = static_cast<size_t>(num_seqs) * HV * kDim * kDim * sizeof(float);
    if (s0 < d0 + bytes && d0 < s0 + bytes) return hipErrorInvalidValue;
  }
  const long long slots = max_slots(total_seq_len, num_seqs);
  if (slots > 0x7fffffffLL || num_seqs > 0x7fffffff - 1) return hipErrorInvalidValue;
  if ((static_cast<long long>(num_seqs) * H + 7) / 8 * 8 * (HV / H) > 0x7fffffffLL)  // scan grid
    return hipErrorInvalidValue;
  if (fixed_scratch) {
    const hipError_t e = current_scratch(&workspace);
    if (e != hipSuccess) return e;
  }

  Params p;
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.state = state;
  p.A_log = A_log;
  p.a = static_cast<const uint16_t*>(a);
  p.dt_bias = dt_bias;
  p.b = static_cast<const uint16_t*>(b);
  p.cu_seqlens = cu_seqlens;
  p.out = static_cast<uint16_t*>(output);
  p.new_state = new_state;
  char* ws = static_cast<char*>(workspace);
  int32_t* offs = reinterpret_cast<int32_t*>(ws);
  i32x4* slot_info = reinterpret_cast<i32x4*>(ws + offsets_bytes(num_seqs));
  p.offs = offs;
  p.slot_info = slot_info;
  p.slots = reinterpret_cast<float*>(ws + offsets_bytes(num_seqs) +
                                     slot_info_bytes(total_seq_len, num_seqs));
  p.seg_chunks = 0;
  p.nseg = 0;
  p.seg_S = p.seg_B = p.seg_M = nullptr;
  if (use_segments(total_seq_len, num_seqs, HV)) {
    char* sg = reinterpret_cast<char*>(p.slots) + slots_bytes(total_seq_len, num_seqs, HV);
    const size_t blocks = seg_blocks_bytes(total_seq_len, num_seqs, HV);
    p.seg_chunks = static_cast<int>(seg_chunks(total_seq_len, num_seqs, HV));
    p.nseg = static_cast<int>(num_segments(total_seq_len, num_seqs, HV));
    p.seg_S = reinterpret_cast<float*>(sg);
    p.seg_B = reinterpret_cast<float*>(sg + blocks);
    p.seg_M = reinterpret_cast<float*>(sg + 2 * blocks);
  }
  p.scale = scale;
  p.L = total_seq_len;
  p.N = num_seqs;
  p.H = H;
  p.HV = HV;
  p.ratio = HV / H;
  p.l2norm = use_qk_l2norm != 0;
  p.single = num_seqs == 1;
  p.few = few_seqs(total_seq_len, num_seqs, HV);
  p.max_slots = slots;
  p.short_limit = maybe_all_short(total_seq_len, num_seqs) ? kSmallTokens : 0;
  p.prep_heads = prep_split(slots, HV) ? 1 : p.ratio;

  hipStream_t stream = static_cast<hipStream_t>(hip_stream);
  // events[i] (optional) is recorded before launch i and events[3] after the last
  auto mark = [&](int i) -> hipError_t {
    return events ? hipEventRecord(static_cast<hipEvent_t>(events[i]), stream) : hipSuccess;
  };
  if (total_seq_len <= kSmallTokens && num_seqs <= 65535) {   // grid z
    // token-by-token path: the three intervals of the timed form are the
    // (empty) offsets and preparation steps and the one launch
    hipError_t e = mark(0);
    if (e == hipSuccess) e = mark(1);
    if (e == hipSuccess) e = mark(2);
    if (e != hipSuccess) return e;
    e = small_prefill(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, output,
                      new_state, total_seq_len, num_seqs, H, HV, use_qk_l2norm != 0, 0, stream);
    if (e == hipSuccess) e = mark(3);
    return e;
  }
  // One workgroup per (sequence or segment role, v-head, column half), in
  // groups of 8 (unit, q/k head) pairs times the GVA ratio times the halves.
  auto scan_grid = [&](long long units, int halves) {
    return dim3(static_cast<unsigned>((units * H + 7) / 8 * 8 * p.ratio * halves));
  };
  if (fused_prefill(total_seq_len, num_seqs, HV)) {
    // one launch (the timed form's intervals as on the token path)
    hipError_t e = mark(0);
    if (e == hipSuccess) e = mark(1);
    if (e == hipSuccess) e = mark(2);
    if (e != hipSuccess) return e;
    p.short_limit = 0;
    constexpr int kHalfW = kScanWaves / 2;
    static_assert(kHalfW == kThreads / 64, "the one-chunk kernel's workgroups are half-state");
    auto* fused = p.l2norm ? one_chunk_kernel<true> : one_chunk_kernel<false>;
    hipLaunchKernelGGL(fused, scan_grid(num_seqs, 2), dim3(kThreads), 0, stream, p);
    e = hipGetLastError();
    if (e == hipSuccess) e = mark(3);
    return e;
  }
  hipError_t e = mark(0);
  if (e != hipSuccess) return e;
  if (p.short_limit > 0) {
    // A batch whose sequences may all be short: the token-by-token kernel
    // first, running only if every sequence has at most kSmallTokens tokens
    // (decided on the device from cu_seqlens); the chunkwise kernels after it
    // return at once in that case and run the whole batch otherwise.
    e = small_prefill(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, output,
                      new_state, total_seq_len, num_seqs, H, HV, use_qk_l2norm != 0,
                      p.short_limit, stream);
    if (e != hipSuccess) return e;
  }
  if (!p.single && !p.few)
    hipLaunchKernelGGL(chunk_offsets_kernel, dim3(1), dim3(kThreads), 0, stream, p, offs,
                       slot_info);
  e = hipGetLastError();
  if (e == hipSuccess) e = mark(1);
  if (e != hipSuccess) return e;
  if (slots > 0) {
    auto* prep = p.few ? prep_kernel<true> : prep_kernel<false>;
    hipLaunchKernelGGL(prep, dim3(static_cast<unsigned>(slots), HV / p.prep_heads),
                       dim3(kThreads), 0, stream, p);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  e = mark(2);
  if (e != hipSuccess) return e;
  if (p.seg_chunks > 0) {
    // segments: transitions and zero-start ends, the starts, then every
    // segment with its outputs (grids: the workspace's segments bound the
    // batch's units; workgroups past them exit)
    auto* scan1 = p.few ? scan_kernel<true, true, false, false, kScanWaves>
                        : scan_kernel<false, true, false, false, kScanWaves>;
    hipLaunchKernelGGL(scan1, scan_grid(seg_units1(p.nseg, num_seqs), 1), dim3(kScanThreads), 0,
                       stream, p);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(seg_combine_kernel,
                       dim3(static_cast<unsigned>(num_seqs * ((HV + 7) & ~7) * 8)),
                       dim3(64 * kCombWaves), 0, stream, p);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    auto* scan = p.few ? (p.l2norm ? scan_kernel<true, true, true, true, kScanWaves>
                                   : scan_kernel<true, true, true, false, kScanWaves>)
                       : (p.l2norm ? scan_kernel<false, true, true, true, kScanWaves>
                                   : scan_kernel<false, true, true, false, kScanWaves>);
    hipLaunchKernelGGL(scan, scan_grid(p.nseg, 1), dim3(kScanThreads), 0, stream, p);
  } else if (half_state_scan(num_seqs, HV)) {
    constexpr int kHalfW = kScanWaves / 2;
    auto* scan = p.few ? (p.l2norm ? scan_kernel<true, false, true, true, kHalfW>
                                   : scan_kernel<true, false, true, false, kHalfW>)
                       : (p.l2norm ? scan_kernel<false, false, true, true, kHalfW>
                                   : scan_kernel<false, false, true, false, kHalfW>);
    hipLaunchKernelGGL(scan, scan_grid(num_seqs, 2), dim3(64 * kHalfW), 0, stream, p);
  } else {
    auto* scan = p.few ? (p.l2norm ? scan_kernel<true, false, true, true, kScanWaves>
                                   : scan_kernel<true, false, true, false, kScanWaves>)
                       : (p.l2norm ? scan_kernel<false, false, true, true, kScanWaves>
                                   : scan_kernel<false, false, true, false, kScanWaves>);
    hipLaunchKernelGGL(scan, scan_grid(num_seqs, 1), dim3(kScanThreads), 0, stream, p);
  }
  e = hipGetLastError();
  if (e == hipSuccess) e = mark(3);
  return e;
}

extern "C" {

size_t gdn_prefill_workspace_bytes(int total_seq_len, int num_seqs, int H, int HV) {
  if (total_seq_len < 0 || num_seqs < 0 || H <= 0 || HV <= 0 || HV % H != 0) return 0;
  return workspace_bytes(total_seq_len, num_seqs, H, HV);
}

int gdn_prefill(const void* q, const void* k, const void* v, const float* state,
                const float* A_log, const void* a, const float* dt_bias, const void* b,
                const int32_t* cu_seqlens, float scale, void* output, float* new_state,
                int total_seq_len, int num_seqs, int H, int HV, int K, int V,
                int use_qk_l2norm, void* workspace, size_t workspace_size,
                void* hip_stream) {
  return prefill_impl(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, output,
                      new_state, total_seq_len, num_seqs, H, HV, K, V, use_qk_l2norm, workspace,
                      workspace_size, hip_stream, nullptr);
}

int gdn_prefill_timed(const void* q, const void* k, const void* v, const float* state,
                      const float* A_log, const void* a, const float* dt_bias, const void* b,
                      const int32_t* cu_seqlens, float scale, void* output, float* new_state,
                      int total_seq_len, int num_seqs, int H, int HV, int K, int V,
                      int use_qk_l2norm, void* workspace, size_t workspace_size,
                      void* hip_stream, void* const* events) {
  if (events == nullptr) return hipErrorInvalidValue;
  for (int i = 0; i < 4; ++i)
    if (events[i] == nullptr) return hipErrorInvalidValue;
  return prefill_impl(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, output,
                      new_state, total_seq_len, num_seqs, H, HV, K, V, use_qk_l2norm, workspace,
                      workspace_size, hip_stream, events);
}

int gdn_prefill_noalloc(const void* q, const void* k, const void* v, const float* state,
                        const float* A_log, const void* a, const float* dt_bias, const void* b,
                        const int32_t* cu_seqlens, float scale, void* output, float* new_state,
                        int total_seq_len, int num_seqs, int H, int HV, int K, int V,
                        int use_qk_l2norm, void* hip_stream) {
  return prefill_impl(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, output,
                      new_state, total_seq_len, num_seqs, H, HV, K, V, use_qk_l2norm, nullptr,
                      0, hip_stream, nullptr, true);
}

int gdn_prefill_token_path_max_tokens(void) { return kSmallTokens; }

int gdn_prefill_dispatches(int total_seq_len, int num_seqs, int HV) {
  if (num_seqs <= 0 || total_seq_len < 0 || HV <= 0) return 0;
  if (total_seq_len <= kSmallTokens && num_seqs <= 65535) return 1;
  if (fused_prefill(total_seq_len, num_seqs, HV)) return 1;
  const int offsets = num_seqs == 1 || few_seqs(total_seq_len, num_seqs, HV) ? 0 : 1;
  const int token = maybe_all_short(total_seq_len, num_seqs) ? 1 : 0;
  if (use_segments(total_seq_len, num_seqs, HV)) return token + offsets + 4;
  return token + offsets + 2;
}

int gdn_prefill_abi_version(void) { return 6; }

}  // extern "C"
