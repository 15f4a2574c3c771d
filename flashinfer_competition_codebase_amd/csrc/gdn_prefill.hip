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
//   W     = T diag(beta e^gamma) K,   U = T diag(beta) V
//   Delta = U - W S_0                  (the per-token delta-rule corrections)
//   O     = scale [diag(e^gamma) Q S_0 + (Q K^T (.) M) Delta],
//           M_ij = e^(gamma_i - gamma_j) for j <= i
//   S_C   = e^(gamma_C) S_0 + (diag(e^(gamma_C - gamma)) K)^T Delta
// Every exponent is <= 0.  With the q/k L2-norm on, the row norms enter as
// per-row scale factors of the same products.
//
// Prefills of at most kSmallTokens (48) tokens in all (so every sequence is
// that short) skip the chunkwise machinery: one launch of the decode kernel's
// variable-length mode (gdn_decode_kernel.h) applies the recurrence token by
// token with the state in registers, one workgroup per (sequence, v-head,
// row tile), reading each sequence's token range from cu_seqlens on the
// device.  Larger prefills run the chunkwise kernels.
//
// Kernels (one stream, in order):
//   1. chunk_offsets: one workgroup turns cu_seqlens into the first chunk
//      slot of every sequence (token ranges clamped to [0, L]) by a scan,
//      and writes each slot's sequence, first token and token count.  With
//      one sequence it is not launched: chunk c is slot c.
//   2. prep, grid (chunk slots, HV), three workgroups per CU: everything
//      that does not depend on the state, for all chunks at once -- gates
//      and gamma, K K^T and Q K^T (bf16 MFMA: the inputs are bf16), T by
//      block recursion (fp32 MFMA), W and U (bf16 MFMA on hi/lo-split T) --
//      into a workspace slot per (chunk, v-head), and K^T and a copy of Q
//      into one per (chunk, q/k head), in the order the scan's MFMAs read
//      them.
//   3. scan, one workgroup per (sequence, v-head, 16- or 32-column slice of
//      the state), XCD-aware order: the sequential part, Delta, O and S_C
//      chunk after chunk (bf16 MFMA on hi/lo-split fp32 operands), the state
//      slice kept in registers and the next chunk's operands loaded while
//      this one runs.
//
// MFMA lane layouts (v_mfma_f32_16x16x4_f32, v_mfma_f32_16x16x32_bf16):
// A[i][k] from lane i + 16 g, B[k][j] from lane j + 16 g (k = g for fp32;
// for bf16 the lane's 8 items cover the 32-long k block), D[i][j] in lane
// j + 16 (i / 4), register i % 4.  A bf16 product sums over its k block in
// any order both operands share; here item e of lane group g stands for
//   k = 16 (e / 4) + 4 g + e % 4,
// so a lane's 8 items are the 4-element runs at k = 4 g and 16 + 4 g, the
// runs a 16 x 16 MFMA result holds per lane -- results become operands
// without exchanging data between lanes.

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
constexpr long long kScanWideHeads = 256;  // N * HV from which the scan takes 32 columns
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
// sequence is longer).  Measured (kernel trace, one sequence): the token loop
// costs ~3.5 us plus ~0.25 us a token, the chunkwise kernels ~15-17 us up to
// 128 tokens at qk4_v8 (16-23 us at qk16_v32); they cross at 45-48 tokens
// (48: 15.1 against 15.4 us at qk4_v8, 17.1 against 16.5 us at qk16_v32).
// Several short sequences favour the token path far more (4 x 12 tokens: 6.8
// against 24.5 us), but past the switch the longest sequence is not known on
// the host.
constexpr int kSmallTokens = 48;
constexpr float kL2Eps = 1e-6f;
constexpr float kSoftplusThreshold = 20.0f;
constexpr float kLn2 = 0.693147180559945309f;

// Workspace slot of one (chunk, v-head), offsets in floats.  The scan's MFMA
// operands (W, P, K^T and a copy of Q) are stored in operand order: a
// 16 x 32 block of an operand is 64 lanes x 8 bf16 contiguous (lane = row +
// 16 g, items in the k order above), so each scan load instruction reads
// 1 KiB contiguous.  fp32 operands are split into a bf16 high and low part
// (x ~ hi + lo to ~2^-16 relative).  U is stored in the MFMA result order
// the scan consumes (per 16 x 16 block, lane-major 4 floats).
constexpr int kBlk = 512;                             // bf16 per 16 x 32 operand block
constexpr int kSlotWh = 0;                            // W hi: blocks (row blk 0..3, k blk 0..3)
constexpr int kSlotWl = kSlotWh + 16 * kBlk / 2;      // W lo
constexpr int kSlotU = kSlotWl + 16 * kBlk / 2;       // U: blocks (row blk 0..3, col blk 0..7)
constexpr int kSlotPh = kSlotU + kChunk * kDim;       // P hi: blocks (row blk 0..3, j blk 0..1),
constexpr int kSlotPl = kSlotPh + 8 * kBlk / 2;       //   P = scale rq_i rk_j M_ij (Q K^T)_ij; lo
constexpr int kSlotQs = kSlotPl + 8 * kBlk / 2;       // scale * rq_i e^gamma_i [64]
constexpr int kSlotKs = kSlotQs + kChunk;             // rk_i e^(gamma_C - gamma_i) [64]
constexpr int kSlotGl = kSlotKs + kChunk;             // e^gamma_C [1], padded to 64
constexpr int kSlotFloats = kSlotGl + 64;
static_assert(kSlotFloats % 64 == 0, "slots stay 256-byte aligned");
// Slot of one (chunk, q/k head), shared by the v-heads of the group: K^T and
// the copy of Q, written by the group's first v-head.
constexpr int kQkSlotKt = 0;                          // K^T: blocks (key blk 0..7, token blk 0..1)
constexpr int kQkSlotQ = kQkSlotKt + 16 * kBlk / 2;   // Q: blocks (token blk 0..3, k blk 0..3)
constexpr int kQkSlotFloats = kQkSlotQ + 16 * kBlk / 2;
static_assert(kQkSlotFloats % 64 == 0, "slots stay 256-byte aligned");

// k (0..31) of item e of lane group g inside a 32-long block.
__host__ __device__ constexpr int k_of(int g, int e) { return 16 * (e >> 2) + 4 * g + (e & 3); }

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

// Operand items of lane group g for k block kb of a bf16 row (k contiguous).
__device__ __forceinline__ s16x8 frag(const uint16_t* row, int kb, int g) {
  return cat(*reinterpret_cast<const s16x4*>(row + 32 * kb + 4 * g),
             *reinterpret_cast<const s16x4*>(row + 32 * kb + 16 + 4 * g));
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
  float* qk_slots;           // [max_slots, H, kQkSlotFloats] (workspace)
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
__device__ __forceinline__ void token_gates(const Params& p, int t, int hv, float& logg,
                                            float& beta) {
  const float x = bf16_to_f32(p.a[static_cast<size_t>(t) * p.HV + hv]) + p.dt_bias[hv];
  const float sp = x > kSoftplusThreshold ? x : __builtin_amdgcn_logf(1.0f + __expf(x)) * kLn2;
  logg = -__expf(p.A_log[hv]) * sp;
  const float bb = bf16_to_f32(p.b[static_cast<size_t>(t) * p.HV + hv]);
  beta = __builtin_amdgcn_rcpf(1.0f + __expf(-bb));
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

// 52 KiB, so that three workgroups share a CU: A (dead once T is built) and
// V (staged from registers after that) share storage, and the 32 x 32
// scratch of the block recursion is T's upper-right quarter, which T never
// uses (rows 0..31, columns 32..63).
struct PrepLds {
  uint16_t K[kChunk * kBfStride];
  union {
    float A[kChunk * kF64Stride];     // strict lower part of (I + A) minus I
    uint16_t V[kChunk * kBfStride];
  };
  float T[kChunk * kF64Stride];       // (I + A)^-1
  float gamma[kChunk];
  float beta[kChunk];
  float rq[kChunk];
  float rk[kChunk];
};
static_assert(sizeof(PrepLds) <= 160 * 1024 / 3, "three preparation workgroups per CU");

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

// FEW: the batch's chunk slots come from cu_seqlens in the kernel (few
// sequences, no offsets kernel); a template flag, so that the kernels of the
// other modes are compiled without that code.
template <bool FEW>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3)))
void prep_kernel(Params p) {
  __shared__ PrepLds lds;
  const int c = blockIdx.x;
  const int hv = blockIdx.y;
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
  const int h = hv / p.ratio;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int col = lane & 15;
  const int g4 = lane >> 4;
  float* slot = p.slots + (static_cast<size_t>(c) * p.HV + hv) * kSlotFloats;
  uint16_t* slot16 = reinterpret_cast<uint16_t*>(slot);
  // the group's first v-head writes the shared Q copy and K^T
  const bool qk_writer = hv == h * p.ratio;
  uint16_t* qk16 =
      reinterpret_cast<uint16_t*>(p.qk_slots + (static_cast<size_t>(c) * p.H + h) * kQkSlotFloats);

  // Every input load of the chunk is issued before the first is waited on.
  u32x4 kreg[4], vreg[4];
  load_rows_bf16(kreg, p.k + (static_cast<size_t>(t0) * p.H + h) * kDim,
                 static_cast<size_t>(p.H) * kDim, n);
  load_rows_bf16(vreg, p.v + (static_cast<size_t>(t0) * p.HV + hv) * kDim,
                 static_cast<size_t>(p.HV) * kDim, n);

  // Q rows 16 wave + col straight into MFMA operand registers (k block m;
  // rows past the chunk's end zero), which are also the scan's
  // operand-ordered copy of Q; with the L2-norm, their row norms.
  s16x8 qa[4];
  const int ra = wave * 16 + col;
  const bool row_ok = ra < n;
  {
    const uint16_t* qrow =
        p.q + ((static_cast<size_t>(t0) + (row_ok ? ra : n - 1)) * p.H + h) * kDim;
#pragma unroll
    for (int m = 0; m < 4; ++m) qa[m] = frag(qrow, m, g4);
  }
  // Gates of token t0 + lane (every wave computes them, wave 0 keeps them);
  // padded rows: no decay, no update.
  float logg, beta;
  token_gates(p, t0 + (lane < n ? lane : n - 1), hv, logg, beta);
  if (lane >= n) logg = beta = 0.0f;

  store_rows_bf16(lds.K, kreg, n);       // V waits in registers until A is dead
  // T's upper blocks that the block recursion multiplies, T_01 and T_23, are
  // zero; the diagonal and lower blocks are all written, the other upper
  // blocks never read.
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int idx = threadIdx.x + it * kThreads;
    const int o = 32 * (idx >> 8);
    lds.T[(o + ((idx >> 4) & 15)) * kF64Stride + o + 16 + (idx & 15)] = 0.0f;
  }
  {
    float sq = 0.0f;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      qa[m] = row_ok ? qa[m] : s16x8{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = bf16_to_f32(static_cast<uint16_t>(qa[m][e]));
        sq = fmaf(x, x, sq);
      }
      if (qk_writer)
        *reinterpret_cast<s16x8*>(qk16 + 2 * kQkSlotQ + (wave * 4 + m) * kBlk + lane * 8) = qa[m];
    }
    sq += __shfl_xor(sq, 16, 64);
    sq += __shfl_xor(sq, 32, 64);
    if (g4 == 0) lds.rq[ra] = p.l2norm ? __builtin_amdgcn_rsqf(sq + kL2Eps) : 1.0f;
  }
  if (wave == 0) {
    float g = logg;                                // inclusive scan over the chunk
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const float y = __shfl_up(g, d, 64);
      if (lane >= d) g += y;
    }
    lds.gamma[lane] = g;
    lds.beta[lane] = beta;
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

  // K K^T for row block `wave` (rows 16 wave .. +15) and (Q K^T)^T = K Q^T
  // for column block `wave`, all 4 blocks of the other index; bf16 MFMA over
  // the 128-long rows.  The transposed product leaves each lane holding 4
  // consecutive j of one row i of P, two of which make the scan's operand
  // items, so P goes out as one 16-byte store per lane and k block.
  {
    f32x4 kk[4], pt[4];
#pragma unroll
    for (int nj = 0; nj < 4; ++nj) {
      kk[nj] = f32x4{0, 0, 0, 0};
      pt[nj] = f32x4{0, 0, 0, 0};
    }
    const int ra = wave * 16 + col;
#pragma unroll
    for (int m = 0; m < kDim / 32; ++m) {
      const s16x8 ak = frag(&lds.K[ra * kBfStride], m, g4);
#pragma unroll
      for (int nj = 0; nj < 4; ++nj) {
        const s16x8 bk = frag(&lds.K[(nj * 16 + col) * kBfStride], m, g4);
        kk[nj] = mfma_bf16(ak, bk, kk[nj]);
        pt[nj] = mfma_bf16(bk, qa[m], pt[nj]);
      }
    }
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
    // P[i][j], i = 16 wave + col, j = 16 nj + 4 g + e
    const int i = wave * 16 + col;
    const float gi = lds.gamma[i];
    const float sqi = p.scale * lds.rq[i];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
      s16x4 hi[2], lo[2];
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int nj = 2 * jb + hf;
        const int j0 = nj * 16 + g4 * 4;
        const f32x4 gj4 = *reinterpret_cast<const f32x4*>(&lds.gamma[j0]);
        const f32x4 rkj4 = *reinterpret_cast<const f32x4*>(&lds.rk[j0]);
        f32x4 pv;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float dec = __expf(fminf(gi - gj4[e], 0.0f));
          const float x = sqi * rkj4[e] * dec * pt[nj][e];
          pv[e] = j0 + e <= i ? x : 0.0f;
        }
        split4(pv, hi[hf], lo[hf]);
      }
      const int bo = (wave * 2 + jb) * kBlk + lane * 8;
      *reinterpret_cast<s16x8*>(slot16 + 2 * kSlotPh + bo) = cat(hi[0], hi[1]);
      *reinterpret_cast<s16x8*>(slot16 + 2 * kSlotPl + bo) = cat(lo[0], lo[1]);
    }
  }
  block_sync_lds();

  // T = (I + A)^-1 by block recursion on 16 x 16 blocks (A is strictly lower
  // triangular, so T is unit lower triangular; the upper blocks stay zero):
  // 1. each wave inverts one diagonal block by forward substitution (one
  //    column per lane, two partial sums per dot product);
  if (lane < 16) {
    const int b0 = wave * 16;
    float t[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float s0 = (r == lane) ? 1.0f : 0.0f, s1 = 0.0f;
#pragma unroll
      for (int j = 0; j < r; ++j) {
        const float aij = lds.A[(b0 + r) * kF64Stride + b0 + j];
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
  store_rows_bf16(lds.V, vreg, n);       // A is dead: V takes its storage
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

  // W = (T diag(beta e^gamma rk)) K (computed transposed, as K^T (T diag)^T,
  // so the result registers are in the scan's operand order) and U =
  // (T diag(beta)) V with bf16 MFMA over 32-token blocks jb: the scaled T is
  // split into hi + lo, K and V are exact bf16.  Wave `wave` computes column
  // tiles 2 wave and 2 wave + 1 (one 32-wide k block of W) for all row
  // blocks; T is lower triangular, so token block 1 only meets row blocks
  // 2 and 3.
  {
    f32x4 w[4][2], u[4][2];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
      for (int q2 = 0; q2 < 2; ++q2) {
        w[rb][q2] = f32x4{0, 0, 0, 0};
        u[rb][q2] = f32x4{0, 0, 0, 0};
      }
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
      s16x8 bk[2], bv[2];
#pragma unroll
      for (int q2 = 0; q2 < 2; ++q2) {
        const int cc = (2 * wave + q2) * 16 + col;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int j = 32 * jb + k_of(g4, e);
          bk[q2][e] = static_cast<short>(lds.K[j * kBfStride + cc]);
          bv[q2][e] = static_cast<short>(lds.V[j * kBfStride + cc]);
        }
      }
      f32x4 xs[2], ys[2];
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int j0 = 32 * jb + 16 * hf + 4 * g4;
        ys[hf] = *reinterpret_cast<const f32x4*>(&lds.beta[j0]);
        const f32x4 gj = *reinterpret_cast<const f32x4*>(&lds.gamma[j0]);
        const f32x4 rkj = *reinterpret_cast<const f32x4*>(&lds.rk[j0]);
#pragma unroll
        for (int e = 0; e < 4; ++e) xs[hf][e] = ys[hf][e] * __expf(gj[e]) * rkj[e];
      }
#pragma unroll
      for (int rb = 2 * jb; rb < 4; ++rb) {
        const float* trow = &lds.T[(rb * 16 + col) * kF64Stride + 32 * jb + 4 * g4];
        s16x4 wh[2], wl[2], uh[2], ul[2];
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          const f32x4 tv = *reinterpret_cast<const f32x4*>(trow + 16 * hf);
          split4(tv * xs[hf], wh[hf], wl[hf]);
          split4(tv * ys[hf], uh[hf], ul[hf]);
        }
        const s16x8 awh = cat(wh[0], wh[1]), awl = cat(wl[0], wl[1]);
        const s16x8 auh = cat(uh[0], uh[1]), aul = cat(ul[0], ul[1]);
#pragma unroll
        for (int q2 = 0; q2 < 2; ++q2) {
          // W^T tile (rows: key index, cols: token), U tile (rows: token)
          w[rb][q2] = mfma_bf16(bk[q2], awh, w[rb][q2]);
          w[rb][q2] = mfma_bf16(bk[q2], awl, w[rb][q2]);
          u[rb][q2] = mfma_bf16(auh, bv[q2], u[rb][q2]);
          u[rb][q2] = mfma_bf16(aul, bv[q2], u[rb][q2]);
        }
      }
    }
    // Lane (col, g) of W^T tile (rb, 2 wave + q2) holds W[16 rb + col][32
    // wave + 16 q2 + 4 g + e]: items 4 q2 + e of the scan's operand block
    // (rb, wave).
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      s16x4 hi[2], lo[2];
#pragma unroll
      for (int q2 = 0; q2 < 2; ++q2) {
        split4(w[rb][q2], hi[q2], lo[q2]);
        *reinterpret_cast<f32x4*>(slot + kSlotU + ((rb * 8 + 2 * wave + q2) * 64 + lane) * 4) =
            u[rb][q2];
      }
      const int bo = (rb * 4 + wave) * kBlk + lane * 8;
      *reinterpret_cast<s16x8*>(slot16 + 2 * kSlotWh + bo) = cat(hi[0], hi[1]);
      *reinterpret_cast<s16x8*>(slot16 + 2 * kSlotWl + bo) = cat(lo[0], lo[1]);
    }
  }

  // Row scales for the scan: Q rows, decayed K rows and the chunk decay.
  if (wave == 1) {
    const float gl = lds.gamma[kChunk - 1];        // padded rows carry gamma forward
    const float gi = lds.gamma[lane];
    slot[kSlotQs + lane] = p.scale * lds.rq[lane] * __expf(gi);
    slot[kSlotKs + lane] = lds.rk[lane] * __expf(gl - gi);
    slot[kSlotGl + lane] = __expf(gl);
  }

  // K^T (A operand of the scan's state update: rows = key index, k =
  // token), in operand order, 16 bytes per store; rows past the chunk's end
  // are zero.  A wave reads 64 consecutive keys of one token row at a time.
  if (!qk_writer) return;                          // uniform per workgroup
#pragma unroll
  for (int it = 0; it < kDim * 8 / kThreads; ++it) {
    const int idx = threadIdx.x + it * kThreads;
    const int kc = idx & (kDim - 1);         // key index 0..127
    const int jg = idx >> 7;                 // token block jb = jg / 4, lane group jg % 4
    s16x8 v8;
#pragma unroll
    for (int e = 0; e < 8; ++e)
      v8[e] = static_cast<short>(lds.K[(32 * (jg >> 2) + k_of(jg & 3, e)) * kBfStride + kc]);
    *reinterpret_cast<s16x8*>(qk16 + 2 * kQkSlotKt + ((kc >> 4) * 2 + (jg >> 2)) * kBlk +
                              ((kc & 15) + 16 * (jg & 3)) * 8) = v8;
  }
}

// ---------------------------------------------------------------------------
// 3. sequential scan over the chunks of a sequence
// ---------------------------------------------------------------------------
// Every product is a bf16 MFMA (16x16x32); fp32 operands enter split into
// hi + lo and a product x y is hi_x hi_y + hi_x lo_y + lo_x hi_y (the lo lo
// term is ~2^-16 relative and dropped); q and k are bf16 already.  The state
// slice and Delta are split once per chunk by the wave that owns them and
// kept transposed in LDS, so every B operand is one 8-byte read.
constexpr int kStStride = kDim + 8;     // S^T rows ([col][k]), bf16
constexpr int kDtStride = kChunk + 8;   // Delta^T and K^T rows, bf16

template <int NT>   // 16-column tiles of the state slice per workgroup
struct ScanLds {
  uint16_t Sh[16 * NT * kStStride];      // state slice^T at the chunk start, hi
  uint16_t Sl[16 * NT * kStStride];      //   lo
  uint16_t Dh[16 * NT * kDtStride];      // Delta^T [col][i], hi
  uint16_t Dl[16 * NT * kDtStride];      //   lo
  uint16_t Eh[16 * NT * kDtStride];      // (ks (.) Delta)^T, hi
  uint16_t El[16 * NT * kDtStride];      //   lo
};

// Per-lane operands of one chunk, loaded ahead of use.
template <int NT>
struct ScanOps {
  s16x8 wh[4], wl[4];   // W rows 16 wave + (lane % 16), k block m (keys)
  s16x8 q[4];           // Q rows (the slot's copy), same k
  s16x8 ph[2], pl[2];   // P rows 16 wave + (lane % 16), k block m (tokens)
  f32x4 u[NT];          // U rows 16 wave + 4 g + e, columns of the NT tiles
  f32x4 ks;             // row scales of the same rows
  float qs;             // output row scale of row 16 wave + (lane % 16)
  float gl;             // chunk decay e^gamma_C
  s16x8 kt[2][2];       // K^T rows 32 wave + 16 t + lane % 16, k block m (tokens)
};

__device__ __forceinline__ s16x8 ld_s16x8(const uint16_t* ptr) {
  return *reinterpret_cast<const s16x8*>(ptr);
}

// Loads of one chunk's operands from its workspace slot.  Every load is
// unconditional and in straight-line code so that the compiler can count the
// loads in flight and wait only for the ones a use needs (a load under a
// branch makes it drain every outstanding load); all of them are 1 KiB
// contiguous wave accesses in the slot's operand order.
template <int NT>
__device__ __forceinline__ void load_w_q_u(const float* slot, const float* qk, int tile0,
                                           int wave, int lane, int g4, ScanOps<NT>& o) {
  const uint16_t* slot16 = reinterpret_cast<const uint16_t*>(slot);
  const uint16_t* qk16 = reinterpret_cast<const uint16_t*>(qk);
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int bo = (wave * 4 + m) * kBlk + lane * 8;
    o.wh[m] = ld_s16x8(slot16 + 2 * kSlotWh + bo);
    o.wl[m] = ld_s16x8(slot16 + 2 * kSlotWl + bo);
    o.q[m] = ld_s16x8(qk16 + 2 * kQkSlotQ + bo);
  }
#pragma unroll
  for (int cq = 0; cq < NT; ++cq)
    o.u[cq] = *reinterpret_cast<const f32x4*>(slot + kSlotU +
                                              ((wave * 8 + tile0 + cq) * 64 + lane) * 4);
  o.ks = *reinterpret_cast<const f32x4*>(slot + kSlotKs + wave * 16 + g4 * 4);
}

template <int NT>
__device__ __forceinline__ void load_p_qs(const float* slot, int wave, int lane,
                                          ScanOps<NT>& o) {
  const uint16_t* slot16 = reinterpret_cast<const uint16_t*>(slot);
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    const int bo = (wave * 2 + m) * kBlk + lane * 8;
    o.ph[m] = ld_s16x8(slot16 + 2 * kSlotPh + bo);
    o.pl[m] = ld_s16x8(slot16 + 2 * kSlotPl + bo);
  }
  o.qs = slot[kSlotQs + wave * 16 + (lane & 15)];
  o.gl = slot[kSlotGl];
}

template <int NT>
__device__ __forceinline__ void load_kt(const float* qk, int wave, int lane, ScanOps<NT>& o) {
  const uint16_t* qk16 = reinterpret_cast<const uint16_t*>(qk);
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int m = 0; m < 2; ++m)
      o.kt[t][m] = ld_s16x8(qk16 + 2 * kQkSlotKt + ((wave * 2 + t) * 2 + m) * kBlk + lane * 8);
  }
}

// One-dimensional grid over (head group of 8, column tile, head in group):
// workgroup b serves head 8 (b / (8 tiles)) + b % 8 and tile (b / 8) % tiles.
// Workgroups are handed to the 8 XCDs round-robin by index, so every tile of
// a head runs on the same XCD (b % 8 is fixed) and the tiles are dispatched
// 8 apart -- together -- sharing that XCD's L2 copy of the chunk operands
// they all read.  Heads past N * HV (padding to a multiple of 8) exit.  FEW
// as for prep_kernel.
template <int NT, bool FEW>
__global__ __launch_bounds__(kThreads) void scan_kernel(Params p) {
  __shared__ ScanLds<NT> lds;
  constexpr int kTiles = 8 / NT;
  const long long b = blockIdx.x;
  const long long head_id = (b / (8 * kTiles)) * 8 + (b & 7);
  if (head_id >= static_cast<long long>(p.N) * p.HV) return;   // uniform per workgroup
  const int s = static_cast<int>(head_id / p.HV);
  const int hv = static_cast<int>(head_id % p.HV);
  const int tile0 = static_cast<int>((b >> 3) % kTiles) * NT;  // first 16-column tile
  const int v0 = tile0 * 16;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int col = lane & 15;
  const int g4 = lane >> 4;
  int start, end;
  seq_range(p, s, start, end);

  // This wave's state tiles: rows k = 32 wave + 16 t + 4 g4 + e, columns
  // v0 + 16 cq + col (k-last storage: 4 consecutive k are one 16-byte vector).
  const size_t head = static_cast<size_t>(s) * p.HV + hv;
  const float* st_in = p.state + head * kDim * kDim;
  float* st_out = p.new_state + head * kDim * kDim;
  f32x4 st[2][NT];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int cq = 0; cq < NT; ++cq) {
      const int kr = wave * 32 + t * 16 + g4 * 4;
      st[t][cq] = (p.state != nullptr && end > start)
                      ? *reinterpret_cast<const f32x4*>(
                            st_in + static_cast<size_t>(v0 + cq * 16 + col) * kDim + kr)
                      : f32x4{0, 0, 0, 0};
    }

  // Chunk count from the slot offsets (never more than the range holds, and
  // never more slots than the workspace has, whatever cu_seqlens contains).
  int slot0, nchunks;
  if (p.single) {
    slot0 = 0;
    nchunks = (end - start + kChunk - 1) / kChunk;
  } else if (FEW) {
    const FewSlots f = few_slots(p);
    slot0 = static_cast<int>(__shfl(f.excl, s, 64));
    nchunks = static_cast<int>(__shfl(f.incl, s, 64)) - slot0;
  } else {
    slot0 = p.offs[s];
    nchunks = p.offs[s + 1] - slot0;
  }
  if (nchunks <= 0) {                 // no tokens: zeros, as the reference
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int cq = 0; cq < NT; ++cq)
        *reinterpret_cast<f32x4*>(st_out + static_cast<size_t>(v0 + cq * 16 + col) * kDim +
                                  wave * 32 + t * 16 + g4 * 4) = f32x4{0, 0, 0, 0};
    return;
  }
  const float* slot_base = p.slots + (static_cast<size_t>(slot0) * p.HV + hv) * kSlotFloats;
  const size_t slot_step = static_cast<size_t>(p.HV) * kSlotFloats;
  const float* qk_base =
      p.qk_slots + (static_cast<size_t>(slot0) * p.H + hv / p.ratio) * kQkSlotFloats;
  const size_t qk_step = static_cast<size_t>(p.H) * kQkSlotFloats;

  ScanOps<NT> op;
  load_kt(qk_base, wave, lane, op);
  load_w_q_u(slot_base, qk_base, tile0, wave, lane, g4, op);
  load_p_qs(slot_base, wave, lane, op);

  for (int ci = 0; ci < nchunks; ++ci) {
    const int t0 = start + ci * kChunk;
    const int n = min(kChunk, end - t0);
    // operands of the next chunk, or of this one again after the last
    const int cn = ci + 1 < nchunks ? ci + 1 : ci;
    const float* slot_next = slot_base + cn * slot_step;
    const float* qk_next = qk_base + cn * qk_step;

    // A. state slice (split) into LDS.  No barrier is needed before these
    // writes: the previous chunk's reads of Sh / Sl (step B) precede its
    // second barrier.
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int cq = 0; cq < NT; ++cq) {
        s16x4 hi, lo;
        split4(st[t][cq], hi, lo);
        const int so = (cq * 16 + col) * kStStride + wave * 32 + t * 16 + g4 * 4;
        *reinterpret_cast<s16x4*>(&lds.Sh[so]) = hi;
        *reinterpret_cast<s16x4*>(&lds.Sl[so]) = lo;
      }
    block_sync_lds();

    // B. Delta rows 16 wave .. +15 = U - W S, and (Q S)^T for the output
    // rows (S^T Q^T: the state fragment is the A operand, Q the B operand);
    // two accumulators per product halve the dependent MFMA chains
    f32x4 ws0[NT], ws1[NT], qs0[NT], qs1[NT];
#pragma unroll
    for (int cq = 0; cq < NT; ++cq) {
      ws0[cq] = ws1[cq] = qs0[cq] = qs1[cq] = f32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) {
#pragma unroll
      for (int cq = 0; cq < NT; ++cq) {
        const int so = (cq * 16 + col) * kStStride;
        const s16x8 sh = frag(&lds.Sh[so], m, g4);
        const s16x8 sl = frag(&lds.Sl[so], m, g4);
        ws0[cq] = mfma_bf16(op.wh[m], sh, ws0[cq]);
        ws1[cq] = mfma_bf16(op.wh[m], sl, ws1[cq]);
        ws0[cq] = mfma_bf16(op.wl[m], sh, ws0[cq]);
        qs0[cq] = mfma_bf16(sh, op.q[m], qs0[cq]);
        qs1[cq] = mfma_bf16(sl, op.q[m], qs1[cq]);
      }
    }
    f32x4 qsum[NT];       // (Q S)^T: lane (row i, g) holds columns 4 g + e
#pragma unroll
    for (int cq = 0; cq < NT; ++cq) {
      const f32x4 ws = ws0[cq] + ws1[cq];
      qsum[cq] = qs0[cq] + qs1[cq];
      f32x4 d, dk;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        d[e] = op.u[cq][e] - ws[e];
        dk[e] = op.ks[e] * d[e];
      }
      s16x4 hi, lo;
      const int dof = (cq * 16 + col) * kDtStride + wave * 16 + g4 * 4;
      split4(d, hi, lo);
      *reinterpret_cast<s16x4*>(&lds.Dh[dof]) = hi;
      *reinterpret_cast<s16x4*>(&lds.Dl[dof]) = lo;
      split4(dk, hi, lo);
      *reinterpret_cast<s16x4*>(&lds.Eh[dof]) = hi;
      *reinterpret_cast<s16x4*>(&lds.El[dof]) = lo;
    }
    load_w_q_u(slot_next, qk_next, tile0, wave, lane, g4, op);
    block_sync_lds();

    // C. output rows, transposed: qs (.) (Q S)^T + Delta^T P^T; lane (row
    // i, g) ends with columns 4 g .. +3 of token row 16 wave + i, stored as
    // one 8-byte piece
    const int orow = wave * 16 + col;
#pragma unroll
    for (int cq = 0; cq < NT; ++cq) {
      f32x4 pd0 = {0, 0, 0, 0}, pd1 = {0, 0, 0, 0};
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const int dof = (cq * 16 + col) * kDtStride;
        const s16x8 dh = frag(&lds.Dh[dof], m, g4);
        const s16x8 dl = frag(&lds.Dl[dof], m, g4);
        pd0 = mfma_bf16(dh, op.ph[m], pd0);
        pd1 = mfma_bf16(dl, op.ph[m], pd1);
        pd0 = mfma_bf16(dh, op.pl[m], pd0);
      }
      const f32x4 pd = pd0 + pd1;
      const float qsc = op.qs;
      const u32x2 ob = {pack_bf16x2(fmaf(qsc, qsum[cq][0], pd[0]), fmaf(qsc, qsum[cq][1], pd[1])),
                        pack_bf16x2(fmaf(qsc, qsum[cq][2], pd[2]), fmaf(qsc, qsum[cq][3], pd[3]))};
      if (orow < n)
        *reinterpret_cast<u32x2*>(p.out + ((static_cast<size_t>(t0) + orow) * p.HV + hv) * kDim +
                                  v0 + cq * 16 + g4 * 4) = ob;
    }

    // D. state rows 32 wave .. +31: S = e^gamma_C S + K^T (ks (.) Delta)
    const float gl = op.gl;
    s16x8 kt[2][2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int m = 0; m < 2; ++m) kt[t][m] = op.kt[t][m];
    load_p_qs(slot_next, wave, lane, op);
    load_kt(qk_next, wave, lane, op);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int cq = 0; cq < NT; ++cq) {
        f32x4 acc0 = st[t][cq] * gl;
        f32x4 acc1 = {0, 0, 0, 0};
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          const int eo = (cq * 16 + col) * kDtStride;
          acc0 = mfma_bf16(kt[t][m], frag(&lds.Eh[eo], m, g4), acc0);
          acc1 = mfma_bf16(kt[t][m], frag(&lds.El[eo], m, g4), acc1);
        }
        st[t][cq] = acc0 + acc1;
      }
  }

#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int cq = 0; cq < NT; ++cq)
      *reinterpret_cast<f32x4*>(st_out + static_cast<size_t>(v0 + cq * 16 + col) * kDim +
                                wave * 32 + t * 16 + g4 * 4) = st[t][cq];
}

bool aligned(const void* ptr, uintptr_t a) {
  return (reinterpret_cast<uintptr_t>(ptr) & (a - 1)) == 0;
}

size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

// Workspace: chunk offsets [N + 1] int32, slot table [max_slots] x 16 bytes,
// the v-head slots [max_slots, HV, kSlotFloats] fp32, then the q/k-head
// slots [max_slots, H, kQkSlotFloats]; each part 256-byte aligned.
size_t offsets_bytes(long long N) { return align256(static_cast<size_t>(N + 1) * sizeof(int32_t)); }

size_t slot_info_bytes(long long L, long long N) {
  return align256(static_cast<size_t>(max_slots(L, N)) * sizeof(i32x4));
}

size_t slots_bytes(long long L, long long N, long long HV) {
  return static_cast<size_t>(max_slots(L, N)) * HV * kSlotFloats * sizeof(float);
}

size_t workspace_bytes(long long L, long long N, long long H, long long HV) {
  return offsets_bytes(N) + slot_info_bytes(L, N) + slots_bytes(L, N, HV) +
         static_cast<size_t>(max_slots(L, N)) * H * kQkSlotFloats * sizeof(float);
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
                                bool l2, hipStream_t stream) {
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
                       h_ratio, 0, A_log, dt_bias, out16, new_state, scale, cu_seqlens, L);
  } else {
    constexpr int kW = 4;
    const dim3 grid(ratio * (kDim / (gdn::kLaneGroups * kNs * kW)), H, N);
    auto* kern = l2 ? gdn::gdn_decode_k128<kNs, kW, true, kPolicy, false, true, true>
                    : gdn::gdn_decode_k128<kNs, kW, false, kPolicy, false, true, true>;
    hipLaunchKernelGGL(kern, grid, dim3(64 * kW), 0, stream, state, q16, k16, v16, a16, b16,
                       h_ratio, 0, A_log, dt_bias, out16, new_state, scale, cu_seqlens, L);
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
  if ((static_cast<long long>(num_seqs) * HV + 7) / 8 * 64 > 0x7fffffffLL)   // scan grid
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
  p.qk_slots = reinterpret_cast<float*>(reinterpret_cast<char*>(p.slots) +
                                        slots_bytes(total_seq_len, num_seqs, HV));
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
                      new_state, total_seq_len, num_seqs, H, HV, use_qk_l2norm != 0, stream);
    if (e == hipSuccess) e = mark(3);
    return e;
  }
  hipError_t e = mark(0);
  if (e != hipSuccess) return e;
  if (!p.single && !p.few)
    hipLaunchKernelGGL(chunk_offsets_kernel, dim3(1), dim3(kThreads), 0, stream, p, offs,
                       slot_info);
  e = hipGetLastError();
  if (e == hipSuccess) e = mark(1);
  if (e != hipSuccess) return e;
  if (slots > 0) {
    auto* prep = p.few ? prep_kernel<true> : prep_kernel<false>;
    hipLaunchKernelGGL(prep, dim3(static_cast<unsigned>(slots), HV), dim3(kThreads), 0,
                       stream, p);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  e = mark(2);
  if (e != hipSuccess) return e;
  // Two 16-column tiles per workgroup once there are enough heads to fill
  // the GPU with them (fewer redundant operand loads); one tile otherwise.
  const long long heads = static_cast<long long>(num_seqs) * HV;
  const long long groups = (heads + 7) / 8;
  if (heads >= kScanWideHeads) {
    auto* scan = p.few ? scan_kernel<2, true> : scan_kernel<2, false>;
    hipLaunchKernelGGL(scan, dim3(static_cast<unsigned>(groups * 8 * 4)), dim3(kThreads), 0,
                       stream, p);
  } else {
    auto* scan = p.few ? scan_kernel<1, true> : scan_kernel<1, false>;
    hipLaunchKernelGGL(scan, dim3(static_cast<unsigned>(groups * 8 * 8)), dim3(kThreads), 0,
                       stream, p);
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
  return num_seqs == 1 || few_seqs(total_seq_len, num_seqs, HV) ? 2 : 3;
}

int gdn_prefill_abi_version(void) { return 6; }

}  // extern "C"
