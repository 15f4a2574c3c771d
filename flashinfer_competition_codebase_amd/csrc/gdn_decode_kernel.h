// gdn_decode_kernel.h - device code of the gfx950 GDN decode kernel
// (included by gdn_decode.hip, which launches it for the decode entry points,
// and by gdn_prefill.hip, which launches its variable-length mode for small
// prefills).  The mapping and the algebra are described in gdn_decode.hip.

#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gdn {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kDim = 128;          // K == V == 128
constexpr int kLaneGroups = 4;     // 16-lane DPP rows per wave64
constexpr float kL2Eps = 1e-6f;    // l2norm: x * rsqrt(sum(x^2) + eps)
constexpr float kSoftplusThreshold = 20.0f;  // torch softplus default
constexpr float kLn2 = 0.693147180559945309f;

// Cache policy for the state stream.
enum : int {
  kPolicyDefault = 0,   // ordinary loads and stores
  kPolicyNtBoth = 1,    // nontemporal state loads and stores
  kPolicyNtStore = 2,   // nontemporal state stores only
  kPolicyNtLoad = 3,    // nontemporal state loads only
};

struct Params {
  const uint16_t* q;        // [B, T, H, 128] bf16
  const uint16_t* k;        // [B, T, H, 128] bf16
  const uint16_t* v;        // [B, T, HV, 128] bf16
  const void* state;        // [B, HV, 128, 128] fp32 or bf16
  const float* A_log;       // [HV]
  const uint16_t* a;        // [B, T, HV] bf16
  const float* dt_bias;     // [HV]
  const uint16_t* b;        // [B, T, HV] bf16
  uint16_t* out;            // [B, T, HV, 128] bf16
  void* new_state;          // [B, HV, 128, 128], may equal state
  float scale;
  int T;                    // tokens per sequence
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
// Two floats to a packed bf16 pair (round to nearest even), lo in the low
// half: one v_cvt_pk_bf16_f32 (two separate conversions would also need a
// v_or to merge the halves).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
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

template <typename V, int POLICY>
__device__ __forceinline__ V load_stream(const void* p) {
  if constexpr (POLICY == kPolicyNtBoth || POLICY == kPolicyNtLoad) {
    return __builtin_nontemporal_load(reinterpret_cast<const V*>(p));
  } else {
    return *reinterpret_cast<const V*>(p);
  }
}

template <typename V, int POLICY>
__device__ __forceinline__ void store_stream(void* p, V x) {
  if constexpr (POLICY == kPolicyNtBoth || POLICY == kPolicyNtStore) {
    __builtin_nontemporal_store(x, reinterpret_cast<V*>(p));
  } else {
    *reinterpret_cast<V*>(p) = x;
  }
}

// The 8 elements lane j owns in a 128-element row, as two 8-byte (fp32
// state layout) or one 16-byte (bf16 state layout) slice of bf16 values.
template <bool BF16>
__device__ __forceinline__ u32x4 load_lane_bf16x8(const uint16_t* row, int j) {
  if constexpr (BF16) {
    return *reinterpret_cast<const u32x4*>(row + 8 * j);
  } else {
    const u32x2 lo = *reinterpret_cast<const u32x2*>(row + 4 * j);
    const u32x2 hi = *reinterpret_cast<const u32x2*>(row + 64 + 4 * j);
    return u32x4{lo.x, lo.y, hi.x, hi.y};
  }
}

__device__ __forceinline__ void unpack_bf16x8(u32x4 w, float (&f)[8]) {
  f[0] = bf16_lo(w.x); f[1] = bf16_hi(w.x);
  f[2] = bf16_lo(w.y); f[3] = bf16_hi(w.y);
  f[4] = bf16_lo(w.z); f[5] = bf16_hi(w.z);
  f[6] = bf16_lo(w.w); f[7] = bf16_hi(w.w);
}

// One state row slice of a lane, as loaded (before conversion to fp32).
template <bool BF16>
struct RowRaw;
template <>
struct RowRaw<false> { f32x4 c[2]; };
template <>
struct RowRaw<true> { u32x4 c; };

template <bool BF16, int POLICY>
__device__ __forceinline__ RowRaw<BF16> load_row(const void* state, size_t row, int j) {
  RowRaw<BF16> r;
  if constexpr (BF16) {
    r.c = load_stream<u32x4, POLICY>(static_cast<const uint16_t*>(state) + row * kDim + 8 * j);
  } else {
    const float* p = static_cast<const float*>(state) + row * kDim + 4 * j;
    r.c[0] = load_stream<f32x4, POLICY>(p);
    r.c[1] = load_stream<f32x4, POLICY>(p + 64);
  }
  return r;
}

template <bool BF16>
__device__ __forceinline__ void unpack_row(const RowRaw<BF16>& r, float (&s)[8]) {
  if constexpr (BF16) {
    unpack_bf16x8(r.c, s);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s[i] = r.c[0][i];
      s[4 + i] = r.c[1][i];
    }
  }
}

template <bool BF16, int POLICY>
__device__ __forceinline__ void store_row(void* state, size_t row, int j, const float (&s)[8]) {
  if constexpr (BF16) {
    const u32x4 w{pack_bf16x2(s[0], s[1]), pack_bf16x2(s[2], s[3]),
                  pack_bf16x2(s[4], s[5]), pack_bf16x2(s[6], s[7])};
    store_stream<u32x4, POLICY>(static_cast<uint16_t*>(state) + row * kDim + 8 * j, w);
  } else {
    float* p = static_cast<float*>(state) + row * kDim + 4 * j;
    store_stream<f32x4, POLICY>(p, f32x4{s[0], s[1], s[2], s[3]});
    store_stream<f32x4, POLICY>(p + 64, f32x4{s[4], s[5], s[6], s[7]});
  }
}

// NS consecutive bf16 values (NS-aligned), as raw bits: one load of 2, 4,
// 8 or 16 bytes.  Kept raw until after the state loads are issued, so that
// no conversion forces a wait on this load before the state stream starts.
template <int NS>
struct Bf16Run;
template <>
struct Bf16Run<1> { uint16_t w; };
template <>
struct Bf16Run<2> { uint32_t w; };
template <>
struct Bf16Run<4> { u32x2 w; };
template <>
struct Bf16Run<8> { u32x4 w; };

template <int NS>
__device__ __forceinline__ Bf16Run<NS> load_bf16_run(const uint16_t* p) {
  Bf16Run<NS> r;
  if constexpr (NS == 1) {
    r.w = *p;
  } else if constexpr (NS == 2) {
    r.w = *reinterpret_cast<const uint32_t*>(p);
  } else if constexpr (NS == 4) {
    r.w = *reinterpret_cast<const u32x2*>(p);
  } else {
    static_assert(NS == 8, "NS must be 1, 2, 4 or 8");
    r.w = *reinterpret_cast<const u32x4*>(p);
  }
  return r;
}

template <int NS>
__device__ __forceinline__ void unpack_bf16_run(const Bf16Run<NS>& r, float (&o)[NS]) {
  if constexpr (NS == 1) {
    o[0] = bf16_bits_to_f32(r.w);
  } else if constexpr (NS == 2) {
    o[0] = bf16_lo(r.w); o[1] = bf16_hi(r.w);
  } else if constexpr (NS == 4) {
    o[0] = bf16_lo(r.w.x); o[1] = bf16_hi(r.w.x);
    o[2] = bf16_lo(r.w.y); o[3] = bf16_hi(r.w.y);
  } else {
    o[0] = bf16_lo(r.w.x); o[1] = bf16_hi(r.w.x);
    o[2] = bf16_lo(r.w.y); o[3] = bf16_hi(r.w.y);
    o[4] = bf16_lo(r.w.z); o[5] = bf16_hi(r.w.z);
    o[6] = bf16_lo(r.w.w); o[7] = bf16_hi(r.w.w);
  }
}

template <int NS>
__device__ __forceinline__ void store_bf16_run(uint16_t* p, const float (&x)[NS]) {
  if constexpr (NS == 1) {
    *p = static_cast<uint16_t>(f32_to_bf16_bits(x[0]));
  } else if constexpr (NS == 2) {
    *reinterpret_cast<uint32_t*>(p) = pack_bf16x2(x[0], x[1]);
  } else if constexpr (NS == 4) {
    *reinterpret_cast<u32x2*>(p) = u32x2{pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3])};
  } else {
    *reinterpret_cast<u32x4*>(p) = u32x4{pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3]),
                                         pack_bf16x2(x[4], x[5]), pack_bf16x2(x[6], x[7])};
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
  // ln(1 + e^x) = log2(1 + e^x) * ln 2; the argument is >= 1, so the raw
  // v_log_f32 needs none of the library's denormal-input scaling.
  const float softplus =
      x > kSoftplusThreshold ? x : __builtin_amdgcn_logf(1.0f + __expf(x)) * kLn2;
  g = __expf(-__expf(A_log) * softplus);
  beta = __builtin_amdgcn_rcpf(1.0f + __expf(-b));
}

// Per-token inputs of one lane, as loaded (raw bits, converted on use).
template <int NS>
struct TokenIn {
  uint16_t a_bits;
  uint16_t b_bits;
  u32x4 q;          // 8 bf16: this lane's elements of q
  u32x4 k;
  Bf16Run<NS> v;    // v of this lane group's NS rows
};

// Inputs of token row bt (the row of q/k/v/a/b: sequence * T + token, or
// the packed row of a variable-length batch).
template <int NS, bool BF16>
__device__ __forceinline__ void load_token(const Params& p, size_t bt, int hq, int hv,
                                           int row0, int j, TokenIn<NS>& in) {
  in.a_bits = p.a[bt * p.HV + hv];
  in.b_bits = p.b[bt * p.HV + hv];
  const size_t qk = (bt * p.H + hq) * kDim;
  in.q = load_lane_bf16x8<BF16>(p.q + qk, j);
  in.k = load_lane_bf16x8<BF16>(p.k + qk, j);
  in.v = load_bf16_run<NS>(p.v + (bt * p.HV + hv) * kDim + row0);
}

// Per-head quantities of one token, from its small inputs only (gates, the
// q/k scales, k.q): they do not depend on the state, so they are computed
// while the state is still in flight.
template <int NS>
struct TokenHead {
  float qf[8];      // this lane's raw q elements
  float kf[8];      // this lane's raw k elements
  float vrow[NS];   // v of the lane group's rows
  float g;          // decay factor
  float beta;
  float kscale;     // 1 / |k| (L2-norm) or 1
  float kq;         // k_hat . q'
  float gk;         // g * kscale
  float gq;         // g * qscale
  float qscale;     // scale / |q| (L2-norm) or scale
};

// The per-head quantities of one token from its q, k, v and its gates.
// Per-head reductions on the raw values: |q|^2, |k|^2 (L2-norm only) and
// k.q.  The normalised, scaled vectors q' = qscale*q and k_hat = kscale*k are
// never formed: their scales multiply the reduced dots instead.
template <int NS, bool L2NORM>
__device__ __forceinline__ void head_of(u32x4 qbits, u32x4 kbits, const Bf16Run<NS>& vbits,
                                        float g, float beta, float scale, TokenHead<NS>& h) {
  unpack_bf16x8(qbits, h.qf);
  unpack_bf16x8(kbits, h.kf);
  unpack_bf16_run<NS>(vbits, h.vrow);
  float qscale = scale;
  float kscale = 1.0f;
  float kq_raw;
  if constexpr (L2NORM) {
    float hs[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      hs[0] = fmaf(h.qf[i], h.qf[i], hs[0]);
      hs[1] = fmaf(h.kf[i], h.kf[i], hs[1]);
      hs[2] = fmaf(h.qf[i], h.kf[i], hs[2]);
    }
    row16_sum<3>(hs);
    // |x|^2 + eps >= eps is a normal number: the raw v_rsq_f32 suffices.
    qscale *= __builtin_amdgcn_rsqf(hs[0] + kL2Eps);
    kscale = __builtin_amdgcn_rsqf(hs[1] + kL2Eps);
    kq_raw = hs[2];
  } else {
    float hs[1] = {0.0f};
#pragma unroll
    for (int i = 0; i < 8; ++i) hs[0] = fmaf(h.qf[i], h.kf[i], hs[0]);
    row16_sum<1>(hs);
    kq_raw = hs[0];
  }
  h.g = g;
  h.beta = beta;
  h.kscale = kscale;
  h.kq = kq_raw * (qscale * kscale);
  h.gk = g * kscale;
  h.gq = g * qscale;
  h.qscale = qscale;
}

template <int NS, bool L2NORM>
__device__ __forceinline__ void token_head(const TokenIn<NS>& in, float A_log, float dt_bias,
                                           float scale, TokenHead<NS>& h) {
  float g, beta;
  gates(bf16_bits_to_f32(in.a_bits), dt_bias, A_log, bf16_bits_to_f32(in.b_bits), g, beta);
  unpack_bf16x8(in.q, h.qf);
  unpack_bf16x8(in.k, h.kf);
  unpack_bf16_run<NS>(in.v, h.vrow);
  float qscale = scale;
  float kscale = 1.0f;
  float kq_raw;
  if constexpr (L2NORM) {
    float hs[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      hs[0] = fmaf(h.qf[i], h.qf[i], hs[0]);
      hs[1] = fmaf(h.kf[i], h.kf[i], hs[1]);
      hs[2] = fmaf(h.qf[i], h.kf[i], hs[2]);
    }
    row16_sum<3>(hs);
    qscale *= __builtin_amdgcn_rsqf(hs[0] + kL2Eps);
    kscale = __builtin_amdgcn_rsqf(hs[1] + kL2Eps);
    kq_raw = hs[2];
  } else {
    float hs[1] = {0.0f};
#pragma unroll
    for (int i = 0; i < 8; ++i) hs[0] = fmaf(h.qf[i], h.kf[i], hs[0]);
    row16_sum<1>(hs);
    kq_raw = hs[0];
  }
  h.g = g;
  h.beta = beta;
  h.kscale = kscale;
  h.kq = kq_raw * (qscale * kscale);
  h.gk = g * kscale;
  h.gq = g * qscale;
  h.qscale = qscale;
}

// Multi-token inputs of one token (its gates come from the per-lane table).
template <int NS>
struct TokenQkv {
  u32x4 q;
  u32x4 k;
  Bf16Run<NS> v;
};

template <int NS, bool BF16>
__device__ __forceinline__ void load_qkv(const Params& p, size_t bt, int hq, int hv, int row0,
                                         int j, TokenQkv<NS>& in) {
  const size_t qk = (bt * p.H + hq) * kDim;
  in.q = load_lane_bf16x8<BF16>(p.q + qk, j);
  in.k = load_lane_bf16x8<BF16>(p.k + qk, j);
  in.v = load_bf16_run<NS>(p.v + (bt * p.HV + hv) * kDim + row0);
}

// Gate table of the multi-token loop: lane l holds the gates of token
// base + l of the sequence (the last token past the end), so each token's
// gates are two lane reads instead of their transcendental chain.
__device__ __forceinline__ float lane_value(float x, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l));
}

struct GateBits {
  uint16_t a;
  uint16_t b;
};

__device__ __forceinline__ GateBits load_gate_bits(const Params& p, size_t tok0, int base, int T,
                                                   int hv, int lane) {
  const int tl = base + lane < T ? base + lane : T - 1;
  const size_t bt = (tok0 + tl) * p.HV + hv;
  return GateBits{p.a[bt], p.b[bt]};
}

// One token of the recurrence on the NS rows a lane group holds: decay,
// delta rule, rank-1 update (in s) and outputs o (reference
// kernel.py:73-75, 101-113).
template <int NS>
__device__ __forceinline__ void token_rows(float (&s)[NS][8], const TokenHead<NS>& h,
                                           float (&o)[NS]) {
  // Per-row reductions k.S and q.S on the undecayed state.
  float red[2 * NS];
#pragma unroll
  for (int n = 0; n < NS; ++n) {
    float ak = 0.0f, aq = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      ak = fmaf(s[n][i], h.kf[i], ak);
      aq = fmaf(s[n][i], h.qf[i], aq);
    }
    red[2 * n] = ak;
    red[2 * n + 1] = aq;
  }
  row16_sum<2 * NS>(red);

#pragma unroll
  for (int n = 0; n < NS; ++n) {
    const float old_v = h.gk * red[2 * n];          // k_hat . (g S)
    const float d = h.beta * (h.vrow[n] - old_v);   // beta * (v - old_v)
    o[n] = fmaf(d, h.kq, h.gq * red[2 * n + 1]);    // q' . S_new
    const float dk = d * h.kscale;                  // S_new = g S + d (x) k_hat
#pragma unroll
    for (int i = 0; i < 8; ++i) s[n][i] = fmaf(dk, h.kf[i], h.g * s[n][i]);
  }
}

// Multi-token form of token_rows with the decay applied lazily.  The lane
// group holds s = S / G, the state divided by the decay G accumulated since
// the last fold (G = 1 at the first token), so a token's decay g costs no
// per-element multiply: with Gn = G g,
//   k_hat . (g S) = Gn kscale (k . s),   q' . S_new = Gn qscale (q . s) + d (k_hat . q')
//   S_new = Gn s + d (x) k_hat  =  Gn (s + (d / Gn) (x) k_hat),
// one FMA per element.  When Gn would fall below kLazyMinDecay (s would
// grow past 2^40 times S, or g itself underflows to 0) the token first
// folds all of it into s -- s = Gn s, after which the token is one with no
// decay on that s (Gn = 1) -- a uniform branch, rare for any decay the
// gates produce.  Only the rounding order differs from token_rows.
constexpr float kLazyMinDecay = 0x1p-40f;

template <int NS>
__device__ __forceinline__ void token_rows_lazy(float (&s)[NS][8], const TokenHead<NS>& h,
                                                float& G, float (&o)[NS]) {
  float gn = G * h.g;                 // decay of S relative to s after this token
  float gk = G * h.gk;                // Gn kscale
  float gq = G * h.gq;                // Gn qscale
  if (gn < kLazyMinDecay) {
#pragma unroll
    for (int n = 0; n < NS; ++n)
#pragma unroll
      for (int i = 0; i < 8; ++i) s[n][i] *= gn;
    gn = 1.0f;
    gk = h.kscale;
    gq = h.qscale;
  }
  float red[2 * NS];
#pragma unroll
  for (int n = 0; n < NS; ++n) {
    float ak = 0.0f, aq = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      ak = fmaf(s[n][i], h.kf[i], ak);
      aq = fmaf(s[n][i], h.qf[i], aq);
    }
    red[2 * n] = ak;
    red[2 * n + 1] = aq;
  }
  row16_sum<2 * NS>(red);

  const float c = h.kscale * __builtin_amdgcn_rcpf(gn);
#pragma unroll
  for (int n = 0; n < NS; ++n) {
    const float d = h.beta * (h.vrow[n] - gk * red[2 * n]);   // beta * (v - k_hat . (g S))
    o[n] = fmaf(d, h.kq, gq * red[2 * n + 1]);              // q' . S_new
    const float dk = d * c;
#pragma unroll
    for (int i = 0; i < 8; ++i) s[n][i] = fmaf(dk, h.kf[i], s[n][i]);
  }
  G = gn;
}

// Block order: consecutive blocks -- which the dispatcher hands round-robin
// to the 8 XCDs -- stream adjacent state rows.  Renumbering blocks so that
// each XCD works on its own contiguous eighth (sharing q/k in that XCD's L2)
// measured 5% slower at B=256 and 18% slower at B=64 (qk16_v32) than this
// natural order, so none is applied.

// T tokens (T = 1 at compile time unless MULTI) of 4*NS*WAVES rows of one
// (b, hv) head per workgroup.  VARLEN (multi-token only): sequence b is the
// token rows [cu_seqlens[b], cu_seqlens[b + 1]) of packed [L, H|HV, ...]
// inputs (the prefill layout), clamped to [0, L]; a sequence with no tokens
// gets a zero state; with short_limit > 0 (at most 64 sequences) the
// workgroups run only if every sequence has at most short_limit tokens.
// MULTI: a null state starts from zeros (the state stream is then only
// written).
//
// The arguments are scalars rather than one struct so that the first 14
// dwords -- every pointer and size the first loads need: six pointers, H and
// HV/H packed into one dword (16 bits each) and T -- are preloaded into
// SGPRs by the dispatcher (-amdgpu-kernarg-preload-count): the state stream
// then starts without waiting for a kernarg memory read.  The remaining
// arguments are read while the first loads are in flight.
//
// The fp32-state multi-token kernels with 2 rows per lane group (launched
// for T = 2 at 65-128 and above 768 heads, for T >= 3 at 65-256 heads) are
// held at 6 waves per SIMD: at their ~71 VGPRs the compiler would allow 7,
// which measured 2.3% slower than 6 at B=256 T=2 (qk16_v32).
// Phase stamps of the instrumented single-token kernel (STAMP): per wave,
// in this order, the real-time clock at entry, the shader clock at entry,
// after the state loads are issued, after the per-head math (the small
// inputs have arrived), when the state has arrived, after the state stores
// are issued, when every store has completed, and the real-time clock at
// the end.
constexpr int kStampsPerWave = 8;

// Clock reads of the instrumented kernel: issued in program order (the
// scheduling barriers), waited for only where the stamps are stored.
__device__ __forceinline__ unsigned long long shader_clock() {
  __builtin_amdgcn_sched_barrier(0);
  const unsigned long long t = __builtin_amdgcn_s_memtime();
  __builtin_amdgcn_sched_barrier(0);
  return t;
}

__device__ __forceinline__ unsigned long long real_clock() {
  __builtin_amdgcn_sched_barrier(0);
  const unsigned long long t = __builtin_amdgcn_s_memrealtime();
  __builtin_amdgcn_sched_barrier(0);
  return t;
}

// A per-head value read through the scalar cache (hv is uniform per
// workgroup): the read the compiler makes of A_log and dt_bias anyway, made
// explicit so that no earlier side effect (the instrumented kernel's clock
// reads count as one) turns it into a vector load queued behind the state
// stream.
__device__ __forceinline__ float scalar_read(const float* ptr) {
  typedef const __attribute__((address_space(4))) float ConstantFloat;
  return *(ConstantFloat*)ptr;  // generic -> constant address space: a C-style cast
}

// This workgroup's place (x, y, z) in a decode grid (row tiles and v-heads
// of a GVA group, q/k head, sequence).  The gridDim.x workgroups of one
// (y, z) all read that sequence's q and k rows of that head, and its gate
// inputs.  Workgroups go to the eight XCDs round-robin in dispatch order (x
// fastest), so in plain order those gridDim.x workgroups land on as many
// XCDs, each fetching the rows from HBM into its own L2 (B=256 qk16_v32
// T=1: 1.016x the algorithmic bytes).  With GROUP (an fp32 state) and the
// host's flag (kGroupFlag in the packed head counts: at least 128 sequences
// in the launch) the workgroups are renumbered: in each
// run of 8 (y, z) groups, dispatch slot L (in the run) runs member L / 8 of
// group L % 8, so a group's workgroups share an XCD (1.0002x; kernel-stamped
// A/B, bitwise identical results: B=128 81.5 -> 80.7 us, B=256 164.1 ->
// 160.3 us, B=512 332.1 -> 321.2 us, T=4 B=256 178.6 -> 177.0 us); a last
// run of fewer than 8 groups keeps the plain order.  Smaller launches and a
// bf16 state keep the plain order: there the renumbering measured no faster
// or slower (B=32: +1%; qk4_v8 B=32 and B=48: +5% and +19%; the fp32 block
// kernel at B=32 and 64: +2%; bf16 state at B=256: even).  The flag rides in
// a preloaded argument: deciding on gridDim, which a workgroup loads from
// the dispatch packet, delayed every small launch's first loads (qk4_v8
// B=48: +6%).
// Power-of-two grid sizes (the usual head counts) take shifts only.
struct GridPos {
  int x, y, z;
};
// Packed head counts of a decode launch: H in bits 0-14, the grouping flag
// in bit 15, the GVA ratio HV / H in bits 16-31.
constexpr unsigned kGroupFlag = 0x8000u;
constexpr long long kGroupMinSeqs = 128;
__host__ __device__ inline int packed_heads(unsigned h_ratio) {
  return static_cast<int>(h_ratio & 0x7fffu);
}
template <bool GROUP>
__device__ __forceinline__ GridPos decode_grid_pos(unsigned h_ratio) {
  if (!GROUP || (h_ratio & kGroupFlag) == 0) {
    return GridPos{static_cast<int>(blockIdx.x), static_cast<int>(blockIdx.y),
                   static_cast<int>(blockIdx.z)};
  }
  const unsigned X = gridDim.x, Y = gridDim.y, Z = gridDim.z;
  const unsigned L = blockIdx.x + X * (blockIdx.y + Y * blockIdx.z);   // < 2^31
  unsigned g, m;
  if (((X & (X - 1)) | (Y & (Y - 1))) == 0) {
    const unsigned lx = __builtin_ctz(X), ly = __builtin_ctz(Y);
    const unsigned run = L >> (lx + 3);
    if (((run + 1) << 3) <= (Z << ly)) {
      g = (run << 3) + (L & 7u);
      m = (L >> 3) & (X - 1);
    } else {
      g = L >> lx;
      m = L & (X - 1);
    }
    return GridPos{static_cast<int>(m), static_cast<int>(g & (Y - 1)), static_cast<int>(g >> ly)};
  }
  const unsigned run = L / (8u * X);
  if (run * 8u + 8u <= Y * Z) {
    g = run * 8u + (L & 7u);
    m = (L >> 3) - run * X;
  } else {
    g = blockIdx.y + Y * blockIdx.z;
    m = blockIdx.x;
  }
  return GridPos{static_cast<int>(m), static_cast<int>(g % Y), static_cast<int>(g / Y)};
}

template <int NS, int WAVES, bool L2NORM, int POLICY, bool BF16, bool MULTI, bool VARLEN,
          bool STAMP>
__device__ __forceinline__ void decode_body(
    const void* state, const uint16_t* q, const uint16_t* k, const uint16_t* v,
    const uint16_t* a, const uint16_t* b, unsigned h_ratio, int T_arg, const float* A_log_p,
    const float* dt_bias_p, uint16_t* out, void* new_state, float scale,
    const int32_t* cu_seqlens, int total_tokens, int short_limit, unsigned long long* stamps) {
  static_assert(MULTI || !VARLEN, "variable-length sequences run the multi-token loop");
  static_assert(!STAMP || (!MULTI && !BF16), "phase stamps: the fp32 single-token kernel");
  unsigned long long st[kStampsPerWave] = {};
  if constexpr (STAMP) {
    st[0] = real_clock();
    st[1] = shader_clock();
  }
  Params p;
  p.state = state;
  p.q = q;
  p.k = k;
  p.v = v;
  p.a = a;
  p.b = b;
  p.A_log = A_log_p;
  p.dt_bias = dt_bias_p;
  p.out = out;
  p.new_state = new_state;
  p.scale = scale;
  p.T = MULTI ? T_arg : 1;
  p.H = packed_heads(h_ratio);
  p.ratio = static_cast<int>(h_ratio >> 16);
  p.HV = p.H * p.ratio;
  constexpr int kRowsPerWave = kLaneGroups * NS;
  constexpr int kRowsPerBlock = kRowsPerWave * WAVES;
  constexpr int kTiles = kDim / kRowsPerBlock;
  static_assert(kDim % kRowsPerBlock == 0, "rows per block must divide 128");
  static_assert((kTiles & (kTiles - 1)) == 0, "tiles per head is a power of two");

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int grp = lane >> 4;
  const int j = lane & 15;

  const GridPos pos = decode_grid_pos<!BF16>(h_ratio);
  const int tile = pos.x & (kTiles - 1);
  const int hq = pos.y;                                  // q/k head
  const int bi = pos.z;
  const int hv = hq * p.ratio + pos.x / kTiles;
  const int head = bi * p.HV + hv;
  const int row0 = tile * kRowsPerBlock + wave * kRowsPerWave + grp * NS;
  const size_t row_base = static_cast<size_t>(head) * kDim + row0;  // state row index
  int T = p.T;
  size_t tok0 = static_cast<size_t>(bi) * T;                        // first token row
  if constexpr (VARLEN) {
    // Clamped to [0, total_tokens]: no cu_seqlens content makes a read
    // leave the inputs.
    int s0 = cu_seqlens[bi];
    int s1 = cu_seqlens[bi + 1];
    s0 = s0 < 0 ? 0 : (s0 > total_tokens ? total_tokens : s0);
    s1 = s1 < s0 ? s0 : (s1 > total_tokens ? total_tokens : s1);
    tok0 = static_cast<size_t>(s0);
    T = s1 - s0;
    if (short_limit > 0) {
      // Only if every sequence of the batch (gridDim.z <= 64 of them) has at
      // most short_limit tokens; else the chunkwise kernels launched after
      // this one run the whole batch.  One read per lane, the same clamping.
      int len = 0;
      if (lane < static_cast<int>(gridDim.z)) {
        int c0 = cu_seqlens[lane];
        int c1 = cu_seqlens[lane + 1];
        c0 = c0 < 0 ? 0 : (c0 > total_tokens ? total_tokens : c0);
        c1 = c1 < c0 ? c0 : (c1 > total_tokens ? total_tokens : c1);
        len = c1 - c0;
      }
      if (__ballot(len > short_limit) != 0) return;      // uniform per block
    }
    if (T == 0) {                      // no tokens: a zero state (uniform per block)
      const float zero[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int n = 0; n < NS; ++n) store_row<BF16, POLICY>(p.new_state, row_base + n, j, zero);
      return;
    }
  }
  // A null state starts from zeros (uniform per launch).  The single-token
  // kernel is never launched with one (the host runs the multi-token loop
  // for T = 1 then), so its state loads stay unconditional.
  const bool has_state = !MULTI || p.state != nullptr;

  // Issue every global load before any arithmetic.  Loads retire in issue
  // order, so the small per-token operands (a, b, q, k, v) go first: their
  // math then overlaps the state stream instead of waiting behind it.  Both
  // bursts use only preloaded arguments; A_log and dt_bias (whose pointers
  // are not preloaded) are read after them, so no wave waits on a kernarg
  // memory read before its state loads are in flight.
  if constexpr (!MULTI) {
    TokenIn<NS> cur;
    load_token<NS, BF16>(p, tok0, hq, hv, row0, j, cur);
    __builtin_amdgcn_sched_barrier(0);

    RowRaw<BF16> raw[NS];
    if (has_state) {
#pragma unroll
      for (int n = 0; n < NS; ++n) raw[n] = load_row<BF16, POLICY>(p.state, row_base + n, j);
    }
    __builtin_amdgcn_sched_barrier(0);
    const float A_log = scalar_read(p.A_log + hv);
    const float dt_bias = scalar_read(p.dt_bias + hv);
    __builtin_amdgcn_sched_barrier(0);  // both reads in flight before either is used
    if constexpr (STAMP) st[2] = shader_clock();

    // The per-head math waits only on the small loads: keep it ahead of
    // everything that waits on the state.
    TokenHead<NS> h;
    token_head<NS, L2NORM>(cur, A_log, dt_bias, p.scale, h);
    // Its scalars are materialised here, ahead of the state: left alone, the
    // compiler sinks the output's factors (scale, the q-norm, k.q) to their
    // use after the state stores, which puts a kernel-argument read and a
    // v_rsq_f32 between the state's arrival and the final output store.
    asm volatile("" ::"v"(h.g), "v"(h.beta), "v"(h.kscale), "v"(h.kq), "v"(h.gk), "v"(h.gq));
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (STAMP) {
      st[3] = shader_clock();
      // a use of the last state load's data: the wait for the whole state
      asm volatile("" ::"v"(raw[NS - 1].c[1][3]));
      st[4] = shader_clock();
    }

    float s[NS][8];
#pragma unroll
    for (int n = 0; n < NS; ++n) {
      if (has_state) {
        unpack_row<BF16>(raw[n], s[n]);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) s[n][i] = 0.0f;
      }
    }
    for (int t = 0; t < T; ++t) {
      float o[NS];
      token_rows<NS>(s, h, o);
      // The state write-back is the kernel's tail: issue it before the output.
#pragma unroll
      for (int n = 0; n < NS; ++n) store_row<BF16, POLICY>(p.new_state, row_base + n, j, s[n]);
      if constexpr (STAMP) st[5] = shader_clock();
      if (j == 0) {
        const size_t out_row = ((tok0 + t) * p.HV + hv) * kDim + row0;
        store_bf16_run<NS>(p.out + out_row, o);
      }
    }
    if constexpr (STAMP) {
      __builtin_amdgcn_s_waitcnt(0);   // every load and store of this wave complete
      st[6] = shader_clock();
      st[7] = real_clock();
      if (lane == 0) {                 // one lane per wave: ordinary vector stores
        const size_t blk = blockIdx.x + static_cast<size_t>(gridDim.x) *
                                             (blockIdx.y + static_cast<size_t>(gridDim.y) * blockIdx.z);
        unsigned long long* dst = stamps + (blk * WAVES + wave) * kStampsPerWave;
#pragma unroll
        for (int i = 0; i < kStampsPerWave; ++i) dst[i] = st[i];
      }
    }
  } else {
    // Multi-token: the state stays in registers across the tokens.  Each
    // lane computes the gates of one token (lane l: token l, tokens 64 and
    // on in further batches of 64) once, and every token reads its two
    // from that table, so a token's instructions are its q/k/v work and the
    // row updates only: with one wave per SIMD, as in small batches and
    // small prefills, a token costs about 4 cycles per instruction.
    TokenQkv<NS> in0;
    load_qkv<NS, BF16>(p, tok0, hq, hv, row0, j, in0);
    GateBits gb = load_gate_bits(p, tok0, 0, T, hv, lane);
    __builtin_amdgcn_sched_barrier(0);

    // The state loads are unconditional: with no state they read new_state
    // (same size, a valid address) and the values are replaced by zeros
    // after the per-head math.  Loads inside a branch would make every later
    // wait for the small inputs assume the branch skipped them, i.e. wait
    // for the whole state before the per-head math.
    const void* src = has_state ? p.state : static_cast<const void*>(p.new_state);
    RowRaw<BF16> raw[NS];
#pragma unroll
    for (int n = 0; n < NS; ++n) raw[n] = load_row<BF16, POLICY>(src, row_base + n, j);
    // Variable-length (small prefill: one wave of few rows per head, latency
    // bound): the inputs of the next kDepth = 3 tokens are in flight while a
    // token is applied, so each load has two tokens' time to arrive; token
    // indices are clamped to the last token, so every load is unconditional
    // (the clamped repeats are never used), and the three input buffers are
    // refilled in place by a loop body unrolled three times.  The decode's
    // multi-token kernels prefetch one token ahead: at large batches deeper
    // prefetch costs registers and load slots (B=256 T=2: 170 -> 202 us),
    // and at small ones it measured no better.
    constexpr int kDepth = VARLEN ? 3 : 1;
    TokenQkv<NS> in1, in2;                    // tokens 1 and 2 (kDepth == 3)
    if constexpr (kDepth == 3) {
      load_qkv<NS, BF16>(p, tok0 + (T > 1 ? 1 : 0), hq, hv, row0, j, in1);
      load_qkv<NS, BF16>(p, tok0 + (T > 2 ? 2 : T - 1), hq, hv, row0, j, in2);
    }
    __builtin_amdgcn_sched_barrier(0);
    const float A_log = p.A_log[hv];
    const float dt_bias = p.dt_bias[hv];
    __builtin_amdgcn_sched_barrier(0);

    float gl, bl;                             // gates of token base + lane
    gates(bf16_bits_to_f32(gb.a), dt_bias, A_log, bf16_bits_to_f32(gb.b), gl, bl);
    TokenHead<NS> h;
    head_of<NS, L2NORM>(in0.q, in0.k, in0.v, lane_value(gl, 0), lane_value(bl, 0), p.scale, h);
    __builtin_amdgcn_sched_barrier(0);

    if (!has_state) {                         // uniform: start from zeros
#pragma unroll
      for (int n = 0; n < NS; ++n) raw[n] = RowRaw<BF16>{};
    }
    float s[NS][8];
#pragma unroll
    for (int n = 0; n < NS; ++n) unpack_row<BF16>(raw[n], s[n]);

    // Per-head quantities of token tt >= 1 (uniform) from its inputs.
    auto head_at = [&](const TokenQkv<NS>& in, int tt) {
      if ((tt & 63) == 0) {                   // tokens tt .. tt + 63: a new gate batch
        gb = load_gate_bits(p, tok0, tt, T, hv, lane);
        gates(bf16_bits_to_f32(gb.a), dt_bias, A_log, bf16_bits_to_f32(gb.b), gl, bl);
      }
      head_of<NS, L2NORM>(in.q, in.k, in.v, lane_value(gl, tt & 63), lane_value(bl, tt & 63),
                          p.scale, h);
    };
    // Token tt with the per-head quantities in h: rows and output.  The
    // state is held divided by the decay G not yet applied to it.
    float G = 1.0f;
    auto apply = [&](int tt) {
      float o[NS];
      token_rows_lazy<NS>(s, h, G, o);
      if (j == 0) store_bf16_run<NS>(p.out + ((tok0 + tt) * p.HV + hv) * kDim + row0, o);
    };

    if constexpr (kDepth == 3) {
      for (int t = 0; t < T; t += 3) {
        load_qkv<NS, BF16>(p, tok0 + (t + 3 < T ? t + 3 : T - 1), hq, hv, row0, j, in0);
        apply(t);
        if (t + 1 >= T) break;
        head_at(in1, t + 1);
        load_qkv<NS, BF16>(p, tok0 + (t + 4 < T ? t + 4 : T - 1), hq, hv, row0, j, in1);
        apply(t + 1);
        if (t + 2 >= T) break;
        head_at(in2, t + 2);
        load_qkv<NS, BF16>(p, tok0 + (t + 5 < T ? t + 5 : T - 1), hq, hv, row0, j, in2);
        apply(t + 2);
        if (t + 3 >= T) break;
        head_at(in0, t + 3);
      }
    } else {
      for (int t = 0; t < T; ++t) {
        TokenQkv<NS> nxt;                     // token t + 1
        if (t + 1 < T) load_qkv<NS, BF16>(p, tok0 + t + 1, hq, hv, row0, j, nxt);
        apply(t);
        if (t + 1 < T) head_at(nxt, t + 1);
      }
    }
#pragma unroll
    for (int n = 0; n < NS; ++n) {
#pragma unroll
      for (int i = 0; i < 8; ++i) s[n][i] *= G;        // the decay still held back
      store_row<BF16, POLICY>(p.new_state, row_base + n, j, s[n]);
    }
  }
}

template <int NS, int WAVES, bool L2NORM, int POLICY, bool BF16, bool MULTI, bool VARLEN>
__global__ __launch_bounds__(64 * WAVES)
__attribute__((amdgpu_waves_per_eu(1, (MULTI && !BF16 && NS == 2) ? 6 : 8))) void gdn_decode_k128(
    const void* state, const uint16_t* q, const uint16_t* k, const uint16_t* v,
    const uint16_t* a, const uint16_t* b, unsigned h_ratio, int T_arg, const float* A_log_p,
    const float* dt_bias_p, uint16_t* out, void* new_state, float scale,
    const int32_t* cu_seqlens, int total_tokens, int short_limit) {
  decode_body<NS, WAVES, L2NORM, POLICY, BF16, MULTI, VARLEN, false>(
      state, q, k, v, a, b, h_ratio, T_arg, A_log_p, dt_bias_p, out, new_state, scale,
      cu_seqlens, total_tokens, short_limit, nullptr);
}

// The fp32 single-token kernel with phase stamps (kStampsPerWave per wave,
// written to `stamps`, indexed by linear block * WAVES + wave): a
// measurement instrument, never launched by the decode entry points.
template <int NS, int WAVES, bool L2NORM>
__global__ __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(1, 8)))
void gdn_decode_k128_stamped(
    const void* state, const uint16_t* q, const uint16_t* k, const uint16_t* v,
    const uint16_t* a, const uint16_t* b, unsigned h_ratio, int T_arg, const float* A_log_p,
    const float* dt_bias_p, uint16_t* out, void* new_state, float scale,
    const int32_t* cu_seqlens, int total_tokens, unsigned long long* stamps) {
  decode_body<NS, WAVES, L2NORM, kPolicyNtBoth, false, false, false, true>(
      state, q, k, v, a, b, h_ratio, T_arg, A_log_p, dt_bias_p, out, new_state, scale,
      cu_seqlens, total_tokens, 0, stamps);
}

}  // namespace gdn
