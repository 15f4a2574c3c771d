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
// Kernels (one stream, in order):
//   1. chunk_offsets: one thread turns cu_seqlens into the first chunk slot
//      of every sequence (token ranges clamped to [0, L]).
//   2. prep, grid (chunk slots, HV): everything that does not depend on the
//      state, for all chunks at once -- gates and gamma, K K^T and Q K^T
//      (bf16 MFMA: the inputs are bf16), T by forward substitution (fp32),
//      W and U (fp32 MFMA) -- into a workspace slot per (chunk, v-head).
//   3. scan, grid (N, HV, 128/16): the sequential part, per sequence, v-head
//      and 16-column slice of the state: Delta, O and S_C chunk after chunk
//      (fp32 MFMA), the state slice kept in registers.
//
// MFMA lane layouts (v_mfma_f32_16x16x4_f32, v_mfma_f32_16x16x16_bf16):
// A[i][k] from lane i + 16 g, B[k][j] from lane j + 16 g (k = g for fp32,
// k = 4 g + e for the bf16 x4 items), D[i][j] in lane j + 16 (i / 4),
// register i % 4.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gdn_prefill.h"

namespace gdn_pf {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kDim = 128;            // K == V == 128
constexpr int kChunk = 64;           // tokens per chunk
constexpr int kThreads = 256;        // 4 wavefronts
constexpr int kVT = 16;              // state columns per scan workgroup
constexpr float kL2Eps = 1e-6f;
constexpr float kSoftplusThreshold = 20.0f;
constexpr float kLn2 = 0.693147180559945309f;

// Workspace slot of one (chunk, v-head), in floats.
constexpr int kSlotW = 0;                          // W [64][128]
constexpr int kSlotU = kSlotW + kChunk * kDim;     // U [64][128]
constexpr int kSlotP = kSlotU + kChunk * kDim;     // scale * rq_i rk_j M_ij (Q K^T)_ij [64][64]
constexpr int kSlotQs = kSlotP + kChunk * kChunk;  // scale * rq_i e^gamma_i [64]
constexpr int kSlotKs = kSlotQs + kChunk;          // rk_i e^(gamma_C - gamma_i) [64]
constexpr int kSlotGl = kSlotKs + kChunk;          // e^gamma_C [1], padded to 64
constexpr int kSlotFloats = kSlotGl + 64;
static_assert(kSlotFloats % 64 == 0, "slots stay 256-byte aligned");

// LDS row strides (elements) chosen so MFMA operand reads spread over banks.
constexpr int kBfStride = kDim + 8;       // bf16 rows of 128
constexpr int kF64Stride = kChunk + 4;    // fp32 rows of 64
constexpr int kF16Stride = kVT + 4;       // fp32 rows of 16

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float x) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));  // round to nearest even
}

__device__ __forceinline__ f32x4 mfma_f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_bf16(s16x4 a, s16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
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
  float* slots;              // [slots, HV, kSlotFloats] (workspace)
  float scale;
  int L;
  int N;
  int H;
  int HV;
  int ratio;                 // HV / H
  int l2norm;
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

// ---------------------------------------------------------------------------
// 1. chunk slots per sequence
// ---------------------------------------------------------------------------
__global__ void chunk_offsets_kernel(Params p, int32_t* offs) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  long long acc = 0;
  offs[0] = 0;
  for (int s = 0; s < p.N; ++s) {
    int start, end;
    seq_range(p, s, start, end);
    acc += (end - start + kChunk - 1) / kChunk;
    if (acc > p.max_slots) acc = p.max_slots;  // cannot happen for clamped ranges
    offs[s + 1] = static_cast<int32_t>(acc);
  }
}

// Sequence owning chunk slot c (offs non-decreasing, offs[0] = 0, c < offs[N]):
// the largest s with offs[s] <= c.
__device__ __forceinline__ int seq_of_slot(const int32_t* offs, int N, int c) {
  int lo = 0, hi = N - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (offs[mid] <= c) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// Gates of token t, v-head hv: log-space decay and beta
// (g = exp(-exp(A_log) softplus(a + dt_bias)), beta = sigmoid(b)).
__device__ __forceinline__ void token_gates(const Params& p, int t, int hv, float& logg,
                                            float& beta) {
  const float x = bf16_to_f32(p.a[static_cast<size_t>(t) * p.HV + hv]) + p.dt_bias[hv];
  const float sp = x > kSoftplusThreshold ? x : __builtin_amdgcn_logf(1.0f + __expf(x)) * kLn2;
  logg = -__expf(p.A_log[hv]) * sp;
  beta = __builtin_amdgcn_rcpf(1.0f + __expf(-bf16_to_f32(p.b[static_cast<size_t>(t) * p.HV + hv])));
}

// Copy rows [0, n) of a [*, stride_rows, 128] bf16 tensor (row r at
// base + r * row_step elements) into LDS rows of kBfStride, zero rows >= n.
__device__ __forceinline__ void stage_rows_bf16(uint16_t* dst, const uint16_t* base,
                                                size_t row_step, int n) {
  // 64 rows x 16 pieces of 16 bytes; 256 threads x 4
  for (int idx = threadIdx.x; idx < kChunk * 16; idx += kThreads) {
    const int r = idx >> 4;
    const int c8 = (idx & 15) * 8;
    u32x4 val = {0u, 0u, 0u, 0u};
    if (r < n) val = *reinterpret_cast<const u32x4*>(base + static_cast<size_t>(r) * row_step + c8);
    uint16_t* d = dst + r * kBfStride + c8;
    *reinterpret_cast<u32x2*>(d) = u32x2{val.x, val.y};
    *reinterpret_cast<u32x2*>(d + 4) = u32x2{val.z, val.w};
  }
}

// ---------------------------------------------------------------------------
// 2. per-chunk preparation
// ---------------------------------------------------------------------------
struct PrepLds {
  uint16_t K[kChunk * kBfStride];
  uint16_t Q[kChunk * kBfStride];
  uint16_t V[kChunk * kBfStride];
  float A[kChunk * kF64Stride];   // strict lower part of (I + A) minus I
  float T[kChunk * kF64Stride];   // (I + A)^-1
  float gamma[kChunk];
  float beta[kChunk];
  float rq[kChunk];
  float rk[kChunk];
};

__global__ __launch_bounds__(kThreads) void prep_kernel(Params p) {
  __shared__ PrepLds lds;
  const int c = blockIdx.x;
  const int hv = blockIdx.y;
  const int nslots = p.offs[p.N];
  if (c >= nslots) return;                         // uniform per workgroup
  const int s = seq_of_slot(p.offs, p.N, c);
  int start, end;
  seq_range(p, s, start, end);
  const int t0 = start + (c - p.offs[s]) * kChunk;
  const int n = min(kChunk, end - t0);             // 1..64
  const int h = hv / p.ratio;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;

  stage_rows_bf16(lds.K, p.k + (static_cast<size_t>(t0) * p.H + h) * kDim,
                  static_cast<size_t>(p.H) * kDim, n);
  stage_rows_bf16(lds.Q, p.q + (static_cast<size_t>(t0) * p.H + h) * kDim,
                  static_cast<size_t>(p.H) * kDim, n);
  stage_rows_bf16(lds.V, p.v + (static_cast<size_t>(t0) * p.HV + hv) * kDim,
                  static_cast<size_t>(p.HV) * kDim, n);
  if (wave == 0) {
    float logg = 0.0f, beta = 0.0f;                // padded rows: no decay, no update
    if (lane < n) token_gates(p, t0 + lane, hv, logg, beta);
    float g = logg;                                // inclusive scan over the chunk
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const float y = __shfl_up(g, d, 64);
      if (lane >= d) g += y;
    }
    lds.gamma[lane] = g;
    lds.beta[lane] = beta;
  }
  __syncthreads();

  // Row scales of the L2-norm (1 when off): 4 threads per row.
  {
    const int r = threadIdx.x >> 2;
    const int part = threadIdx.x & 3;
    float sq = 0.0f, sk = 0.0f;
    if (p.l2norm) {
      for (int i = part * 32; i < part * 32 + 32; ++i) {
        const float x = bf16_to_f32(lds.Q[r * kBfStride + i]);
        const float y = bf16_to_f32(lds.K[r * kBfStride + i]);
        sq = fmaf(x, x, sq);
        sk = fmaf(y, y, sk);
      }
      sq += __shfl_xor(sq, 1, 64);
      sk += __shfl_xor(sk, 1, 64);
      sq += __shfl_xor(sq, 2, 64);
      sk += __shfl_xor(sk, 2, 64);
    }
    if (part == 0) {
      lds.rq[r] = p.l2norm ? __builtin_amdgcn_rsqf(sq + kL2Eps) : 1.0f;
      lds.rk[r] = p.l2norm ? __builtin_amdgcn_rsqf(sk + kL2Eps) : 1.0f;
    }
  }
  __syncthreads();

  float* slot = p.slots + (static_cast<size_t>(c) * p.HV + hv) * kSlotFloats;
  const int col = lane & 15;
  const int g4 = lane >> 4;

  // K K^T and Q K^T for row block `wave` (rows 16 wave .. +15), all 4 column
  // blocks; bf16 MFMA over the 128-long rows.
  {
    f32x4 kk[4], qk[4];
#pragma unroll
    for (int nj = 0; nj < 4; ++nj) {
      kk[nj] = f32x4{0, 0, 0, 0};
      qk[nj] = f32x4{0, 0, 0, 0};
    }
    const int ra = wave * 16 + col;
#pragma unroll
    for (int ks = 0; ks < kDim / 16; ++ks) {
      const int kk0 = ks * 16 + g4 * 4;
      const s16x4 ak = *reinterpret_cast<const s16x4*>(&lds.K[ra * kBfStride + kk0]);
      const s16x4 aq = *reinterpret_cast<const s16x4*>(&lds.Q[ra * kBfStride + kk0]);
#pragma unroll
      for (int nj = 0; nj < 4; ++nj) {
        const s16x4 bk = *reinterpret_cast<const s16x4*>(&lds.K[(nj * 16 + col) * kBfStride + kk0]);
        kk[nj] = mfma_bf16(ak, bk, kk[nj]);
        qk[nj] = mfma_bf16(aq, bk, qk[nj]);
      }
    }
#pragma unroll
    for (int nj = 0; nj < 4; ++nj) {
      const int j = nj * 16 + col;
      const float gj = lds.gamma[j];
      const float rkj = lds.rk[j];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = wave * 16 + g4 * 4 + e;
        const float gi = lds.gamma[i];
        const float dec = j <= i ? __expf(gi - gj) : 0.0f;   // exponent <= 0
        const float a = j < i ? lds.beta[i] * dec * lds.rk[i] * rkj * kk[nj][e] : 0.0f;
        lds.A[i * kF64Stride + j] = a;
        slot[kSlotP + i * kChunk + j] = p.scale * lds.rq[i] * rkj * dec * qk[nj][e];
      }
    }
  }
  __syncthreads();

  // T = (I + A)^-1 by forward substitution, one column per lane of wave 0:
  // T[i][c] = delta_ic - sum_{j<i} A[i][j] T[j][c].
  if (wave == 0) {
    float tc[kChunk];
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
      float acc = (i == lane) ? 1.0f : 0.0f;
#pragma unroll
      for (int j = 0; j < i; ++j) acc = fmaf(-lds.A[i * kF64Stride + j], tc[j], acc);
      tc[i] = acc;
      lds.T[i * kF64Stride + lane] = acc;
    }
  }
  __syncthreads();

  // W = T diag(beta e^gamma rk) K and U = T diag(beta) V, row block `wave`
  // (T is lower triangular: inner index j < 16 (wave + 1)), fp32 MFMA.
  {
    const int ra = wave * 16 + col;
    f32x4 w[8], u[8];
#pragma unroll
    for (int nj = 0; nj < 8; ++nj) {
      w[nj] = f32x4{0, 0, 0, 0};
      u[nj] = f32x4{0, 0, 0, 0};
    }
    const int ksteps = 4 * (wave + 1);
    for (int ks = 0; ks < ksteps; ++ks) {
      const int j = ks * 4 + g4;
      const float ta = lds.T[ra * kF64Stride + j];
      const float xs = lds.beta[j] * __expf(lds.gamma[j]) * lds.rk[j];
      const float ys = lds.beta[j];
#pragma unroll
      for (int nj = 0; nj < 8; ++nj) {
        const int cc = nj * 16 + col;
        w[nj] = mfma_f32(ta, xs * bf16_to_f32(lds.K[j * kBfStride + cc]), w[nj]);
        u[nj] = mfma_f32(ta, ys * bf16_to_f32(lds.V[j * kBfStride + cc]), u[nj]);
      }
    }
#pragma unroll
    for (int nj = 0; nj < 8; ++nj) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = wave * 16 + g4 * 4 + e;
        slot[kSlotW + i * kDim + nj * 16 + col] = w[nj][e];
        slot[kSlotU + i * kDim + nj * 16 + col] = u[nj][e];
      }
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
}

// ---------------------------------------------------------------------------
// 3. sequential scan over the chunks of a sequence
// ---------------------------------------------------------------------------
struct ScanLds {
  uint16_t K[kChunk * kBfStride];     // K rows of the chunk
  float S[kDim * kF16Stride];         // state slice S[k][v] at the chunk start
  float D[kChunk * kF16Stride];       // Delta [64][16]
  float ks[kChunk];
};

__global__ __launch_bounds__(kThreads) void scan_kernel(Params p) {
  __shared__ ScanLds lds;
  const int s = blockIdx.x;
  const int hv = blockIdx.y;
  const int v0 = blockIdx.z * kVT;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int col = lane & 15;
  const int g4 = lane >> 4;
  const int h = hv / p.ratio;
  int start, end;
  seq_range(p, s, start, end);

  // This wave's two 16-row tiles of the state slice: rows k = 32 wave + 16 t
  // + 4 g4 + e, column v0 + col.  k-last storage: 4 consecutive k are one
  // 16-byte vector.
  const size_t head = static_cast<size_t>(s) * p.HV + hv;
  float* ns_base = p.new_state + head * kDim * kDim + static_cast<size_t>(v0 + col) * kDim;
  f32x4 st[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int kr = wave * 32 + t * 16 + g4 * 4;
    st[t] = (p.state != nullptr && end > start)
                ? *reinterpret_cast<const f32x4*>(p.state + head * kDim * kDim +
                                                 static_cast<size_t>(v0 + col) * kDim + kr)
                : f32x4{0, 0, 0, 0};
  }

  // Chunk count from the slot offsets (never more than the range holds, and
  // never more slots than the workspace has, whatever cu_seqlens contains).
  const int nchunks = p.offs[s + 1] - p.offs[s];
  for (int ci = 0; ci < nchunks; ++ci) {
    const int t0 = start + ci * kChunk;
    const int n = min(kChunk, end - t0);
    const float* slot = p.slots + (static_cast<size_t>(p.offs[s] + ci) * p.HV + hv) * kSlotFloats;

    // state slice and K rows into LDS
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        lds.S[(wave * 32 + t * 16 + g4 * 4 + e) * kF16Stride + col] = st[t][e];
    }
    stage_rows_bf16(lds.K, p.k + (static_cast<size_t>(t0) * p.H + h) * kDim,
                    static_cast<size_t>(p.H) * kDim, n);
    if (threadIdx.x < kChunk) lds.ks[threadIdx.x] = slot[kSlotKs + threadIdx.x];
    __syncthreads();

    // Delta rows 16 wave .. +15 = U - W S;  O rows = Qs Q S (+ P Delta below)
    const int ra = wave * 16 + col;                // A-operand row of this lane
    const bool row_ok = ra < n;
    const float qs = slot[kSlotQs + ra];
    const uint16_t* qrow = p.q + ((static_cast<size_t>(t0) + (row_ok ? ra : 0)) * p.H + h) * kDim;
    f32x4 ws = {0, 0, 0, 0};
    f32x4 qsacc = {0, 0, 0, 0};
#pragma unroll 4
    for (int m = 0; m < kDim / 16; ++m) {
      // inner index k = 16 m + 4 g4 + e for step e: one 16-byte W load and
      // one 8-byte Q load per lane per m
      const int kb = m * 16 + g4 * 4;
      const f32x4 wv = *reinterpret_cast<const f32x4*>(slot + kSlotW + ra * kDim + kb);
      u32x2 qv = {0u, 0u};
      if (row_ok) qv = *reinterpret_cast<const u32x2*>(qrow + kb);
      const float qf[4] = {bf16_to_f32(static_cast<uint16_t>(qv.x & 0xffffu)),
                           bf16_to_f32(static_cast<uint16_t>(qv.x >> 16)),
                           bf16_to_f32(static_cast<uint16_t>(qv.y & 0xffffu)),
                           bf16_to_f32(static_cast<uint16_t>(qv.y >> 16))};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float sb = lds.S[(kb + e) * kF16Stride + col];
        ws = mfma_f32(wv[e], sb, ws);
        qsacc = mfma_f32(qs * qf[e], sb, qsacc);
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = wave * 16 + g4 * 4 + e;
      lds.D[i * kF16Stride + col] = slot[kSlotU + i * kDim + v0 + col] - ws[e];
    }
    __syncthreads();

    // O rows += P Delta; store
    {
      f32x4 o = qsacc;
#pragma unroll 4
      for (int m = 0; m < kChunk / 16; ++m) {
        const int kb = m * 16 + g4 * 4;
        const f32x4 pv = *reinterpret_cast<const f32x4*>(slot + kSlotP + ra * kChunk + kb);
#pragma unroll
        for (int e = 0; e < 4; ++e) o = mfma_f32(pv[e], lds.D[(kb + e) * kF16Stride + col], o);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = wave * 16 + g4 * 4 + e;
        if (i < n)
          p.out[((static_cast<size_t>(t0) + i) * p.HV + hv) * kDim + v0 + col] = f32_to_bf16(o[e]);
      }
    }

    // S rows 32 wave .. +31: S = e^gamma_C S + (ks (.) K)^T Delta
    {
      const float gl = slot[kSlotGl];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        f32x4 acc = st[t] * gl;
        const int kr = wave * 32 + t * 16 + col;   // A-operand row (state row k)
#pragma unroll 4
        for (int m = 0; m < kChunk / 16; ++m) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int i = m * 16 + g4 * 4 + e;
            const float ak = lds.ks[i] * bf16_to_f32(lds.K[i * kBfStride + kr]);
            acc = mfma_f32(ak, lds.D[i * kF16Stride + col], acc);
          }
        }
        st[t] = acc;
      }
    }
    __syncthreads();   // LDS is rewritten by the next chunk
  }

#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int kr = wave * 32 + t * 16 + g4 * 4;
    *reinterpret_cast<f32x4*>(ns_base + kr) = st[t];
  }
}

bool aligned(const void* ptr, uintptr_t a) {
  return (reinterpret_cast<uintptr_t>(ptr) & (a - 1)) == 0;
}

size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

long long max_slots(long long L, long long N) { return (L + kChunk - 1) / kChunk + N; }

size_t offsets_bytes(long long N) { return align256(static_cast<size_t>(N + 1) * sizeof(int32_t)); }

size_t workspace_bytes(long long L, long long N, long long HV) {
  return offsets_bytes(N) +
         static_cast<size_t>(max_slots(L, N)) * HV * kSlotFloats * sizeof(float);
}

}  // namespace gdn_pf

using namespace gdn_pf;

extern "C" {

size_t gdn_prefill_workspace_bytes(int total_seq_len, int num_seqs, int HV) {
  if (total_seq_len < 0 || num_seqs < 0 || HV <= 0) return 0;
  return workspace_bytes(total_seq_len, num_seqs, HV);
}

int gdn_prefill(const void* q, const void* k, const void* v, const float* state,
                const float* A_log, const void* a, const float* dt_bias, const void* b,
                const int32_t* cu_seqlens, float scale, void* output, float* new_state,
                int total_seq_len, int num_seqs, int H, int HV, int K, int V,
                int use_qk_l2norm, void* workspace, size_t workspace_size,
                void* hip_stream) {
  if (total_seq_len < 0 || num_seqs < 0 || H <= 0 || HV <= 0 || HV % H != 0)
    return hipErrorInvalidValue;
  if (K != kDim || V != kDim) return hipErrorInvalidValue;
  if (HV > 65535) return hipErrorInvalidValue;      // grid y
  if (num_seqs == 0) return hipSuccess;
  if (!cu_seqlens || !A_log || !dt_bias || !new_state || !workspace)
    return hipErrorInvalidValue;
  if (total_seq_len > 0 && (!q || !k || !v || !a || !b || !output))
    return hipErrorInvalidValue;
  if (workspace_size < workspace_bytes(total_seq_len, num_seqs, HV)) return hipErrorInvalidValue;
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
  p.offs = static_cast<const int32_t*>(workspace);
  p.slots = reinterpret_cast<float*>(static_cast<char*>(workspace) + offsets_bytes(num_seqs));
  p.scale = scale;
  p.L = total_seq_len;
  p.N = num_seqs;
  p.H = H;
  p.HV = HV;
  p.ratio = HV / H;
  p.l2norm = use_qk_l2norm != 0;
  p.max_slots = slots;

  hipStream_t stream = static_cast<hipStream_t>(hip_stream);
  hipLaunchKernelGGL(chunk_offsets_kernel, dim3(1), dim3(64), 0, stream, p,
                     static_cast<int32_t*>(workspace));
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (slots > 0) {
    hipLaunchKernelGGL(prep_kernel, dim3(static_cast<unsigned>(slots), HV), dim3(kThreads), 0,
                       stream, p);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(scan_kernel, dim3(num_seqs, HV, kDim / kVT), dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

int gdn_prefill_abi_version(void) { return 1; }

}  // extern "C"
