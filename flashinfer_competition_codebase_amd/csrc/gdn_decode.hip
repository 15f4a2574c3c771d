// gdn_decode.hip - Gated Delta Net single-token decode step for gfx950.
//
// One fused kernel per step: gate math, optional q/k L2-norm, state decay,
// delta-rule correction, rank-1 update and output mat-vec, reading and
// writing the contiguous k-last fp32 state [B, HV, V=128, K=128] in place
// (or into a second buffer).  Semantics follow the reference's decode step
// (solution/triton/kernel.py:72-118, fused form kernel.py:289-335).
//
// Work mapping (wave64):
//   * one state row (128 fp32 = 512 B) is owned by one 16-lane DPP row of a
//     wavefront; lane j holds elements [4j, 4j+4) and [64+4j, 64+4j+4), so
//     each of the two 128-bit loads of a row reads 256 contiguous bytes;
//   * a wavefront holds 4 lane groups x NS rows each (NS "slots"), i.e. it
//     keeps 4*NS*512 B of state in flight per load burst;
//   * a workgroup of WAVES wavefronts covers 4*NS*WAVES consecutive rows of
//     one (b, hv) head; a head is split over T = 128/(4*NS*WAVES) workgroups;
//   * grid (ratio*T, H, B) with ratio = HV/H: x = (v-head within its GVA
//     group, row tile), y = q/k head, z = batch.  Every index is a shift or
//     a multiply-add (no integer division before the first load), and the
//     x-fastest dispatch order walks the state in memory order.
//   * dot products over K reduce inside the 16-lane row with four DPP adds
//     (quad_perm xor1, quad_perm xor2, row_half_mirror, row_mirror), so no
//     LDS or cross-row traffic is needed.
//
// The two per-row reductions of the reference (k.S before the update, then
// q.S_new after it) are made independent:  with S_new = g*S + d (x) k,
//   q.S_new = g*(q.S) + d*(k.q),   d = beta*(v - g*(k.S)),
// so k.S and q.S reduce together and k.q is one per-head reduction.  This
// only reorders fp32 rounding.

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gdn_decode.h"

namespace gdn {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kDim = 128;          // K == V == 128
constexpr int kLaneGroups = 4;     // 16-lane DPP rows per wave64
constexpr float kL2Eps = 1e-6f;    // l2norm: x * rsqrt(sum(x^2) + eps)
constexpr float kSoftplusThreshold = 20.0f;  // torch softplus default

// Cache policy for the state stream.
enum : int {
  kPolicyDefault = 0,   // ordinary loads and stores
  kPolicyNtBoth = 1,    // nontemporal state loads and stores
  kPolicyNtStore = 2,   // nontemporal state stores only
  kPolicyNtLoad = 3,    // nontemporal state loads only
};

struct Params {
  const uint16_t* q;        // [B, H, 128] bf16
  const uint16_t* k;        // [B, H, 128] bf16
  const uint16_t* v;        // [B, HV, 128] bf16
  const float* state;       // [B, HV, 128, 128] fp32
  const float* A_log;       // [HV]
  const uint16_t* a;        // [B, HV] bf16
  const float* dt_bias;     // [HV]
  const uint16_t* b;        // [B, HV] bf16
  uint16_t* out;            // [B, HV, 128] bf16
  float* new_state;         // [B, HV, 128, 128] fp32, may equal state
  float scale;
  int H;
  int HV;
  int ratio;                // HV / H
};

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}
// Round-to-nearest-even fp32 -> bf16 (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float x) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(x)));
}

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(
      __builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}

// Sum over each 16-lane DPP row; every lane of the row ends with the same
// bits (each step adds a value to its mirror, and fp32 add commutes).
template <int N>
__device__ __forceinline__ void row16_sum(float (&x)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) x[i] += dpp<0xB1>(x[i]);   // quad_perm [1,0,3,2]
#pragma unroll
  for (int i = 0; i < N; ++i) x[i] += dpp<0x4E>(x[i]);   // quad_perm [2,3,0,1]
#pragma unroll
  for (int i = 0; i < N; ++i) x[i] += dpp<0x141>(x[i]);  // row_half_mirror
#pragma unroll
  for (int i = 0; i < N; ++i) x[i] += dpp<0x140>(x[i]);  // row_mirror
}

template <int POLICY>
__device__ __forceinline__ f32x4 load_state(const float* p) {
  if constexpr (POLICY == kPolicyNtBoth || POLICY == kPolicyNtLoad) {
    return __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
  } else {
    return *reinterpret_cast<const f32x4*>(p);
  }
}

template <int POLICY>
__device__ __forceinline__ void store_state(float* p, f32x4 x) {
  if constexpr (POLICY == kPolicyNtBoth || POLICY == kPolicyNtStore) {
    __builtin_nontemporal_store(x, reinterpret_cast<f32x4*>(p));
  } else {
    *reinterpret_cast<f32x4*>(p) = x;
  }
}

// NS consecutive bf16 values starting at an NS-aligned element.
template <int NS>
__device__ __forceinline__ void load_bf16_run(const uint16_t* p, float (&o)[NS]) {
  if constexpr (NS == 1) {
    o[0] = bf16_bits_to_f32(*p);
  } else if constexpr (NS == 2) {
    const uint32_t w = *reinterpret_cast<const uint32_t*>(p);
    o[0] = bf16_lo(w);
    o[1] = bf16_hi(w);
  } else if constexpr (NS == 4) {
    const u32x2 w = *reinterpret_cast<const u32x2*>(p);
    o[0] = bf16_lo(w.x); o[1] = bf16_hi(w.x);
    o[2] = bf16_lo(w.y); o[3] = bf16_hi(w.y);
  } else {
    static_assert(NS == 8, "NS must be 1, 2, 4 or 8");
    const u32x4 w = *reinterpret_cast<const u32x4*>(p);
    o[0] = bf16_lo(w.x); o[1] = bf16_hi(w.x);
    o[2] = bf16_lo(w.y); o[3] = bf16_hi(w.y);
    o[4] = bf16_lo(w.z); o[5] = bf16_hi(w.z);
    o[6] = bf16_lo(w.w); o[7] = bf16_hi(w.w);
  }
}

template <int NS>
__device__ __forceinline__ void store_bf16_run(uint16_t* p, const float (&x)[NS]) {
  uint32_t h[NS];
#pragma unroll
  for (int i = 0; i < NS; ++i) h[i] = f32_to_bf16_bits(x[i]);
  if constexpr (NS == 1) {
    *p = static_cast<uint16_t>(h[0]);
  } else if constexpr (NS == 2) {
    *reinterpret_cast<uint32_t*>(p) = h[0] | (h[1] << 16);
  } else if constexpr (NS == 4) {
    u32x2 w;
    w.x = h[0] | (h[1] << 16);
    w.y = h[2] | (h[3] << 16);
    *reinterpret_cast<u32x2*>(p) = w;
  } else {
    u32x4 w;
    w.x = h[0] | (h[1] << 16);
    w.y = h[2] | (h[3] << 16);
    w.z = h[4] | (h[5] << 16);
    w.w = h[6] | (h[7] << 16);
    *reinterpret_cast<u32x4*>(p) = w;
  }
}

// Decay and update gates from the raw per-head inputs:
//   g = exp(-exp(A_log) * softplus(a + dt_bias)),  beta = sigmoid(b),
// softplus(x) = x for x > 20 else log(1 + exp(x)) (torch's threshold).
// Uses the native v_exp_f32 / v_log_f32 / v_rcp_f32 instructions: the gate
// is a handful of scalars per head, and the relative error these add (a few
// 1e-7 times the exponent's magnitude) is far inside the state tolerance.
__device__ __forceinline__ void gates(float a, float dt_bias, float A_log,
                                      float b, float& g, float& beta) {
  const float x = a + dt_bias;
  const float softplus = x > kSoftplusThreshold ? x : __logf(1.0f + __expf(x));
  g = __expf(-__expf(A_log) * softplus);
  beta = __builtin_amdgcn_rcpf(1.0f + __expf(-b));
}

__device__ __forceinline__ void unpack4(u32x2 w, float* f) {
  f[0] = bf16_lo(w.x); f[1] = bf16_hi(w.x);
  f[2] = bf16_lo(w.y); f[3] = bf16_hi(w.y);
}

// Block order: consecutive blocks -- which the dispatcher hands round-robin
// to the 8 XCDs -- stream adjacent state rows.  Renumbering blocks so that
// each XCD works on its own contiguous eighth (sharing q/k in that XCD's L2)
// measured 5% slower at B=256 and 18% slower at B=64 (qk16_v32) than this
// natural order, so none is applied.

// One decode step for 4*NS*WAVES rows of one (b, hv) head per workgroup.
template <int NS, int WAVES, bool L2NORM, int POLICY>
__global__ __launch_bounds__(64 * WAVES) void gdn_decode_k128(Params p) {
  constexpr int kRowsPerWave = kLaneGroups * NS;
  constexpr int kRowsPerBlock = kRowsPerWave * WAVES;
  constexpr int kTiles = kDim / kRowsPerBlock;
  static_assert(kDim % kRowsPerBlock == 0, "rows per block must divide 128");

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int grp = lane >> 4;
  const int j = lane & 15;

  static_assert((kTiles & (kTiles - 1)) == 0, "tiles per head is a power of two");
  const int tile = static_cast<int>(blockIdx.x) & (kTiles - 1);
  const int hq = static_cast<int>(blockIdx.y);          // q/k head
  const int bi = static_cast<int>(blockIdx.z);
  const int hv = hq * p.ratio + static_cast<int>(blockIdx.x) / kTiles;
  const int head = bi * p.HV + hv;
  const int row0 = tile * kRowsPerBlock + wave * kRowsPerWave + grp * NS;

  // Issue every global load before any arithmetic.  Loads retire in issue
  // order, so the small per-head operands (gate scalars, q, k, v) go first:
  // their math then overlaps the state stream instead of waiting behind it.
  const float A_log = p.A_log[hv];
  const float dt_bias = p.dt_bias[hv];
  const uint16_t a_bits = p.a[head];
  const uint16_t b_bits = p.b[head];

  const size_t qk_off = (static_cast<size_t>(bi) * p.H + hq) * kDim + 4 * j;
  const u32x2 qa = *reinterpret_cast<const u32x2*>(p.q + qk_off);
  const u32x2 qb = *reinterpret_cast<const u32x2*>(p.q + qk_off + 64);
  const u32x2 ka = *reinterpret_cast<const u32x2*>(p.k + qk_off);
  const u32x2 kb = *reinterpret_cast<const u32x2*>(p.k + qk_off + 64);

  const size_t row_base = static_cast<size_t>(head) * kDim + row0;  // row index
  float vrow[NS];
  load_bf16_run<NS>(p.v + row_base, vrow);
  __builtin_amdgcn_sched_barrier(0);

  const float* sp = p.state + row_base * kDim + 4 * j;
  f32x4 s[NS][2];
#pragma unroll
  for (int n = 0; n < NS; ++n) {
    s[n][0] = load_state<POLICY>(sp + n * kDim);
    s[n][1] = load_state<POLICY>(sp + n * kDim + 64);
  }
  __builtin_amdgcn_sched_barrier(0);

  // Gates (uniform per head), reference kernel.py:73-75 / 289-305.
  float g, beta;
  gates(bf16_bits_to_f32(a_bits), dt_bias, A_log, bf16_bits_to_f32(b_bits), g, beta);

  float qf[8], kf[8];
  unpack4(qa, qf);
  unpack4(qb, qf + 4);
  unpack4(ka, kf);
  unpack4(kb, kf + 4);

  // Per-head reductions: |q|^2, |k|^2 (L2-norm only) and k.q.
  float qscale = p.scale;
  float kscale = 1.0f;
  float kq;
  if constexpr (L2NORM) {
    float hs[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      hs[0] = fmaf(qf[i], qf[i], hs[0]);
      hs[1] = fmaf(kf[i], kf[i], hs[1]);
      hs[2] = fmaf(qf[i], kf[i], hs[2]);
    }
    row16_sum<3>(hs);
    const float iq = rsqrtf(hs[0] + kL2Eps);
    kscale = rsqrtf(hs[1] + kL2Eps);
    qscale *= iq;
    kq = hs[2] * (qscale * kscale);
  } else {
    float hs[1] = {0.0f};
#pragma unroll
    for (int i = 0; i < 8; ++i) hs[0] = fmaf(qf[i], kf[i], hs[0]);
    row16_sum<1>(hs);
    kq = hs[0] * qscale;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    qf[i] *= qscale;  // q' = scale * q_hat
    kf[i] *= kscale;  // k_hat
  }

  // Per-row reductions k_hat.S and q'.S on the undecayed state.
  float red[2 * NS];
#pragma unroll
  for (int n = 0; n < NS; ++n) {
    float ak = 0.0f, aq = 0.0f;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ak = fmaf(s[n][c][i], kf[4 * c + i], ak);
        aq = fmaf(s[n][c][i], qf[4 * c + i], aq);
      }
    }
    red[2 * n] = ak;
    red[2 * n + 1] = aq;
  }
  row16_sum<2 * NS>(red);

  // Delta rule, rank-1 update and output (reference kernel.py:101-113).
  float o[NS];
#pragma unroll
  for (int n = 0; n < NS; ++n) {
    const float old_v = g * red[2 * n];             // k_hat . (g S)
    const float d = beta * (vrow[n] - old_v);       // beta * (v - old_v)
    o[n] = fmaf(d, kq, g * red[2 * n + 1]);         // q' . S_new
#pragma unroll
    for (int c = 0; c < 2; ++c) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        s[n][c][i] = fmaf(d, kf[4 * c + i], g * s[n][c][i]);
      }
    }
  }

  if (j == 0) store_bf16_run<NS>(p.out + row_base, o);
  float* dp = p.new_state + row_base * kDim + 4 * j;
#pragma unroll
  for (int n = 0; n < NS; ++n) {
    store_state<POLICY>(dp + n * kDim, s[n][0]);
    store_state<POLICY>(dp + n * kDim + 64, s[n][1]);
  }
}

// ---------------------------------------------------------------------------
// Host side: validation, launch-shape choice and template dispatch.
// ---------------------------------------------------------------------------

// Launch bundle: stream plus optional events that hipExtLaunchKernelGGL
// stamps with the kernel's own start and end timestamps.
struct Launch {
  hipStream_t stream;
  hipEvent_t start;
  hipEvent_t stop;
};

template <int NS, int W, bool L2, int POL>
hipError_t launch_one(const Params& p, unsigned blocks, const Launch& l) {
  constexpr unsigned kT = kDim / (kLaneGroups * NS * W);
  const unsigned per_batch = static_cast<unsigned>(p.HV) * kT;
  const dim3 grid_xyz(static_cast<unsigned>(p.ratio) * kT, static_cast<unsigned>(p.H),
                      blocks / per_batch);
  if (l.start || l.stop) {
    hipExtLaunchKernelGGL((gdn_decode_k128<NS, W, L2, POL>), grid_xyz,
                          dim3(64 * W), 0, l.stream, l.start, l.stop, 0, p);
  } else {
    hipLaunchKernelGGL((gdn_decode_k128<NS, W, L2, POL>), grid_xyz,
                       dim3(64 * W), 0, l.stream, p);
  }
  return hipGetLastError();
}

template <int NS, int W, bool L2>
hipError_t by_policy(int pol, const Params& p, unsigned blocks, const Launch& s) {
  switch (pol) {
    case kPolicyDefault: return launch_one<NS, W, L2, kPolicyDefault>(p, blocks, s);
    case kPolicyNtBoth: return launch_one<NS, W, L2, kPolicyNtBoth>(p, blocks, s);
    case kPolicyNtStore: return launch_one<NS, W, L2, kPolicyNtStore>(p, blocks, s);
    case kPolicyNtLoad: return launch_one<NS, W, L2, kPolicyNtLoad>(p, blocks, s);
    default: return hipErrorInvalidValue;
  }
}

template <int NS, int W>
hipError_t by_norm(bool l2, int pol, const Params& p, unsigned blocks, const Launch& s) {
  return l2 ? by_policy<NS, W, true>(pol, p, blocks, s)
            : by_policy<NS, W, false>(pol, p, blocks, s);
}

template <int NS>
hipError_t by_waves(int w, bool l2, int pol, const Params& p, unsigned blocks,
                    const Launch& s) {
  switch (w) {
    case 1: return by_norm<NS, 1>(l2, pol, p, blocks, s);
    case 2: return by_norm<NS, 2>(l2, pol, p, blocks, s);
    case 4: return by_norm<NS, 4>(l2, pol, p, blocks, s);
    case 8:
      if constexpr (NS * 8 <= 32) return by_norm<NS, 8>(l2, pol, p, blocks, s);
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
}

hipError_t dispatch(int ns, int w, bool l2, int pol, const Params& p,
                    unsigned blocks, const Launch& s) {
  switch (ns) {
    case 1: return by_waves<1>(w, l2, pol, p, blocks, s);
    case 2: return by_waves<2>(w, l2, pol, p, blocks, s);
    case 4: return by_waves<4>(w, l2, pol, p, blocks, s);
    case 8: return by_waves<8>(w, l2, pol, p, blocks, s);
    default: return hipErrorInvalidValue;
  }
}

bool is_pow2_upto8(int x) { return x == 1 || x == 2 || x == 4 || x == 8; }

bool aligned(const void* p, uintptr_t a) {
  return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

// Launch shape for B*HV heads, from a rocprofv3 sweep of every shape and
// cache policy on MI355X: two rows per lane group with nontemporal state
// loads and stores is fastest from B*HV = 256 (B=8 qk16_v32, 7.0 us) to
// 8192 (B=256, 168 us = 6.4 TB/s); below that every shape sits within
// 0.1 us of a fixed ~3 us launch-plus-round-trip floor.
void choose_shape(long long heads, int* ns, int* waves, int* policy) {
  *ns = 2;
  *policy = kPolicyNtBoth;
  *waves = heads <= 64 ? 2 : 4;  // 16 or 32 rows per block
}

int step_impl(const void* q, const void* k, const void* v, const float* state,
              const float* A_log, const void* a, const float* dt_bias,
              const void* b, float scale, void* output, float* new_state,
              int B, int H, int HV, int K, int V, int use_qk_l2norm, int ns,
              int waves, int policy, void* start_event, void* stop_event,
              void* hip_stream) {
  if (B < 0 || H <= 0 || HV <= 0 || HV % H != 0) return hipErrorInvalidValue;
  if (H > 65535) return hipErrorInvalidValue;  // grid y
  if (K != kDim || V != kDim) return hipErrorInvalidValue;
  if (!is_pow2_upto8(ns) || !is_pow2_upto8(waves) || ns * waves > 32)
    return hipErrorInvalidValue;
  if (policy < kPolicyDefault || policy > kPolicyNtLoad) return hipErrorInvalidValue;
  if (B == 0) return hipSuccess;
  if (!q || !k || !v || !state || !A_log || !a || !dt_bias || !b || !output ||
      !new_state)
    return hipErrorInvalidValue;
  // 16-byte state rows chunks, 8-byte q/k chunks, up to 16-byte v/out runs.
  if (!aligned(state, 16) || !aligned(new_state, 16) || !aligned(q, 8) ||
      !aligned(k, 8) || !aligned(v, 16) || !aligned(output, 16) ||
      !aligned(A_log, 4) || !aligned(dt_bias, 4) || !aligned(a, 2) ||
      !aligned(b, 2))
    return hipErrorInvalidValue;
  const size_t state_bytes =
      static_cast<size_t>(B) * HV * kDim * kDim * sizeof(float);
  if (new_state != state) {
    const uintptr_t s0 = reinterpret_cast<uintptr_t>(state);
    const uintptr_t d0 = reinterpret_cast<uintptr_t>(new_state);
    if (s0 < d0 + state_bytes && d0 < s0 + state_bytes)
      return hipErrorInvalidValue;  // partial overlap: only exact aliasing
  }

  const int rows_per_block = kLaneGroups * ns * waves;
  const long long tiles = kDim / rows_per_block;
  const long long threads_per_block = 64LL * waves;
  // Keep each launch's work-item count well inside 32 bits.
  const long long max_blocks = (1LL << 31) / threads_per_block;
  long long batches_per_launch = max_blocks / (tiles * HV);
  if (batches_per_launch > 65535) batches_per_launch = 65535;  // grid z limit
  if (batches_per_launch < 1) return hipErrorInvalidValue;

  Params p;
  p.A_log = A_log;
  p.dt_bias = dt_bias;
  p.scale = scale;
  p.H = H;
  p.HV = HV;
  p.ratio = HV / H;
  for (long long b0 = 0; b0 < B; b0 += batches_per_launch) {
    const long long nb = (B - b0) < batches_per_launch ? (B - b0) : batches_per_launch;
    p.q = static_cast<const uint16_t*>(q) + b0 * H * kDim;
    p.k = static_cast<const uint16_t*>(k) + b0 * H * kDim;
    p.v = static_cast<const uint16_t*>(v) + b0 * HV * kDim;
    p.state = state + b0 * HV * kDim * kDim;
    p.a = static_cast<const uint16_t*>(a) + b0 * HV;
    p.b = static_cast<const uint16_t*>(b) + b0 * HV;
    p.out = static_cast<uint16_t*>(output) + b0 * HV * kDim;
    p.new_state = new_state + b0 * HV * kDim * kDim;
    const unsigned blocks = static_cast<unsigned>(nb * HV * tiles);
    // Start stamp on the first launch, stop stamp on the last.
    Launch l;
    l.stream = static_cast<hipStream_t>(hip_stream);
    l.start = b0 == 0 ? static_cast<hipEvent_t>(start_event) : nullptr;
    l.stop = b0 + nb == B ? static_cast<hipEvent_t>(stop_event) : nullptr;
    const hipError_t e = dispatch(ns, waves, use_qk_l2norm != 0, policy, p, blocks, l);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace gdn

using namespace gdn;

extern "C" {

int gdn_decode_step(const void* q, const void* k, const void* v,
                    const float* state, const float* A_log, const void* a,
                    const float* dt_bias, const void* b, float scale,
                    void* output, float* new_state, int B, int H, int HV,
                    int K, int V, int use_qk_l2norm, void* hip_stream) {
  if (B < 0 || HV <= 0) return hipErrorInvalidValue;
  int ns = 0, waves = 0, policy = 0;
  choose_shape(static_cast<long long>(B) * HV, &ns, &waves, &policy);
  return step_impl(q, k, v, state, A_log, a, dt_bias, b, scale, output,
                   new_state, B, H, HV, K, V, use_qk_l2norm, ns, waves,
                   policy, nullptr, nullptr, hip_stream);
}

int gdn_decode_step_shaped(const void* q, const void* k, const void* v,
                           const float* state, const float* A_log,
                           const void* a, const float* dt_bias, const void* b,
                           float scale, void* output, float* new_state, int B,
                           int H, int HV, int K, int V, int use_qk_l2norm,
                           int rows_per_lane_group, int waves_per_block,
                           int cache_policy, void* start_event,
                           void* stop_event, void* hip_stream) {
  return step_impl(q, k, v, state, A_log, a, dt_bias, b, scale, output,
                   new_state, B, H, HV, K, V, use_qk_l2norm,
                   rows_per_lane_group, waves_per_block, cache_policy,
                   start_event, stop_event, hip_stream);
}

int gdn_decode_launch_shape(int B, int HV, int* rows_per_lane_group,
                            int* waves_per_block, int* cache_policy,
                            long long* num_blocks) {
  if (B < 0 || HV <= 0 || !rows_per_lane_group || !waves_per_block ||
      !cache_policy || !num_blocks)
    return hipErrorInvalidValue;
  int ns = 0, waves = 0, policy = 0;
  choose_shape(static_cast<long long>(B) * HV, &ns, &waves, &policy);
  *rows_per_lane_group = ns;
  *waves_per_block = waves;
  *cache_policy = policy;
  *num_blocks = static_cast<long long>(B) * HV * (kDim / (kLaneGroups * ns * waves));
  return hipSuccess;
}

const char* gdn_decode_error_string(int code) {
  return hipGetErrorString(static_cast<hipError_t>(code));
}

int gdn_decode_abi_version(void) { return 1; }

}  // extern "C"
