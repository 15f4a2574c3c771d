// gdn_decode.hip - Gated Delta Net decode step for gfx950 (MI355X).
//
// One fused kernel per call: gate math, optional q/k L2-norm, state decay,
// delta-rule correction, rank-1 update and output mat-vec, reading and
// writing the contiguous k-last state [B, HV, V=128, K=128] in place (or
// into a second buffer).  Semantics follow the reference's decode step
// (solution/triton/kernel.py:72-118, fused form kernel.py:289-335); T > 1
// tokens per sequence apply that step token after token against the state
// kept in registers (the per-token recurrence of
// solution/triton/prefill_kernel.py:144-178), and the state may be stored
// as fp32 (the reference's) or bf16 (fp32 arithmetic either way).
//
// The kernel's device code is in gdn_decode_kernel.h (shared with the
// prefill library, which runs its variable-length mode for small prefills)
// and, for T = 2..4 tokens at the head counts where it is faster, in
// gdn_decode_block.h (the tokens applied as one block on the matrix cores);
// this file is the host side: validation, launch-shape tables, template
// dispatch and the C ABI.
//
// Work mapping (wave64):
//   * one state row (128 elements) is owned by one 16-lane DPP row of a
//     wavefront, 8 elements per lane: for an fp32 state lane j holds
//     [4j, 4j+4) and [64+4j, 64+4j+4), so each of the row's two 128-bit
//     loads reads 256 contiguous bytes; for a bf16 state lane j holds
//     [8j, 8j+8), one 128-bit load over the 256-byte row;
//   * a wavefront holds 4 lane groups x NS rows each (NS "slots");
//   * a workgroup of WAVES wavefronts covers 4*NS*WAVES consecutive rows of
//     one (b, hv) head; a head is split over R = 128/(4*NS*WAVES) workgroups;
//   * grid (ratio*R, H, B) with ratio = HV/H: x = (v-head within its GVA
//     group, row tile), y = q/k head, z = batch.  Every index is a shift or
//     a multiply-add (no integer division before the first load), and the
//     x-fastest dispatch order walks the state in memory order -- except in
//     launches of 128 or more sequences with an fp32 state, whose workgroups
//     are renumbered so that those of one (sequence, q/k head) share an XCD
//     (decode_grid_pos; shifts for power-of-two grid sizes);
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

#include <new>

#include "gdn_decode.h"
#include "gdn_decode_block.h"
#include "gdn_decode_kernel.h"

namespace gdn {

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

// Kernel variant: the fp32 single-token kernel is built for every launch
// shape and cache policy (the sweep space); bf16-state and multi-token
// kernels for every launch shape with policies 0 and 1.
struct Variant {
  bool l2;
  bool bf16;
  bool multi;
};

// Launch shapes: rows_per_lane_group 1, 2, 4 or 8 runs the token-by-token
// kernel (a wave holds 4 lane groups of that many rows); 16, 32 or 64 runs
// the block kernel for T = 2..4 (a wave holds that many rows, as 16-row MFMA
// tiles).
bool is_block_shape(int ns) { return ns == 16 || ns == 32 || ns == 64; }
int rows_per_wave(int ns) { return is_block_shape(ns) ? ns : kLaneGroups * ns; }

template <int NS, int W, int POL, bool BF16, bool MULTI>
hipError_t launch_one(bool l2, const Params& p, unsigned nb, const Launch& l) {
  constexpr unsigned kT = kDim / (kLaneGroups * NS * W);
  const dim3 grid(static_cast<unsigned>(p.ratio) * kT, static_cast<unsigned>(p.H), nb);
  const dim3 block(64 * W);
  auto* kern = l2 ? gdn_decode_k128<NS, W, true, POL, BF16, MULTI, false>
                  : gdn_decode_k128<NS, W, false, POL, BF16, MULTI, false>;
  const int32_t* no_seqlens = nullptr;
  // H below 2^15 and HV/H below 2^16 (checked by the caller); the grouping
  // flag for launches of many sequences
  const unsigned h_ratio = static_cast<unsigned>(p.H) | (static_cast<unsigned>(p.ratio) << 16) |
                           (nb >= kGroupMinSeqs ? kGroupFlag : 0u);
  if (l.start || l.stop) {
    hipExtLaunchKernelGGL(kern, grid, block, 0, l.stream, l.start, l.stop, 0, p.state, p.q,
                          p.k, p.v, p.a, p.b, h_ratio, p.T, p.A_log, p.dt_bias, p.out,
                          p.new_state, p.scale, no_seqlens, 0, 0);
  } else {
    hipLaunchKernelGGL(kern, grid, block, 0, l.stream, p.state, p.q, p.k, p.v, p.a, p.b,
                       h_ratio, p.T, p.A_log, p.dt_bias, p.out, p.new_state, p.scale,
                       no_seqlens, 0, 0);
  }
  return hipGetLastError();
}

template <int NS, int W, bool BF16, bool MULTI>
hipError_t by_policy(int pol, bool l2, const Params& p, unsigned nb, const Launch& l) {
  constexpr bool kFull = !BF16 && !MULTI;
  switch (pol) {
    case kPolicyDefault: return launch_one<NS, W, kPolicyDefault, BF16, MULTI>(l2, p, nb, l);
    case kPolicyNtBoth: return launch_one<NS, W, kPolicyNtBoth, BF16, MULTI>(l2, p, nb, l);
    case kPolicyNtStore:
      if constexpr (kFull) return launch_one<NS, W, kPolicyNtStore, BF16, MULTI>(l2, p, nb, l);
      return hipErrorInvalidValue;
    case kPolicyNtLoad:
      if constexpr (kFull) return launch_one<NS, W, kPolicyNtLoad, BF16, MULTI>(l2, p, nb, l);
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
}

template <int NS, bool BF16, bool MULTI>
hipError_t by_waves(int w, int pol, bool l2, const Params& p, unsigned nb, const Launch& l) {
  switch (w) {
    case 1: return by_policy<NS, 1, BF16, MULTI>(pol, l2, p, nb, l);
    case 2: return by_policy<NS, 2, BF16, MULTI>(pol, l2, p, nb, l);
    case 4: return by_policy<NS, 4, BF16, MULTI>(pol, l2, p, nb, l);
    case 8:
      if constexpr (NS * 8 <= 32) return by_policy<NS, 8, BF16, MULTI>(pol, l2, p, nb, l);
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
}

template <bool BF16, bool MULTI>
hipError_t by_ns(int ns, int w, int pol, bool l2, const Params& p, unsigned nb,
                 const Launch& l) {
  switch (ns) {
    case 1: return by_waves<1, BF16, MULTI>(w, pol, l2, p, nb, l);
    case 2: return by_waves<2, BF16, MULTI>(w, pol, l2, p, nb, l);
    case 4: return by_waves<4, BF16, MULTI>(w, pol, l2, p, nb, l);
    case 8: return by_waves<8, BF16, MULTI>(w, pol, l2, p, nb, l);
    default: return hipErrorInvalidValue;
  }
}

// Block kernel (gdn_decode_block.h): R tiles of 16 rows per wave.
template <int R, int W, bool BF16>
hipError_t launch_block(bool l2, const Params& p, unsigned nb, const Launch& l) {
  constexpr unsigned kT = kDim / (16 * R * W);
  const dim3 grid(static_cast<unsigned>(p.ratio) * kT, static_cast<unsigned>(p.H), nb);
  const dim3 block(64 * W);
  auto* kern = l2 ? gdn_decode_block<R, W, true, BF16> : gdn_decode_block<R, W, false, BF16>;
  const unsigned h_ratio = static_cast<unsigned>(p.H) | (static_cast<unsigned>(p.ratio) << 16) |
                           (nb >= kGroupMinSeqs ? kGroupFlag : 0u);
  if (l.start || l.stop) {
    hipExtLaunchKernelGGL(kern, grid, block, 0, l.stream, l.start, l.stop, 0, p.state, p.q,
                          p.k, p.v, p.a, p.b, h_ratio, p.T, p.A_log, p.dt_bias, p.out,
                          p.new_state, p.scale);
  } else {
    hipLaunchKernelGGL(kern, grid, block, 0, l.stream, p.state, p.q, p.k, p.v, p.a, p.b,
                       h_ratio, p.T, p.A_log, p.dt_bias, p.out, p.new_state, p.scale);
  }
  return hipGetLastError();
}

template <bool BF16>
hipError_t dispatch_block(int rows, int w, bool l2, const Params& p, unsigned nb,
                          const Launch& l) {
  switch (rows * 16 + w) {
    case 16 * 16 + 1: return launch_block<1, 1, BF16>(l2, p, nb, l);
    case 16 * 16 + 2: return launch_block<1, 2, BF16>(l2, p, nb, l);
    case 16 * 16 + 4: return launch_block<1, 4, BF16>(l2, p, nb, l);
    case 16 * 16 + 8: return launch_block<1, 8, BF16>(l2, p, nb, l);
    case 32 * 16 + 1: return launch_block<2, 1, BF16>(l2, p, nb, l);
    case 32 * 16 + 2: return launch_block<2, 2, BF16>(l2, p, nb, l);
    case 32 * 16 + 4: return launch_block<2, 4, BF16>(l2, p, nb, l);
    case 64 * 16 + 1: return launch_block<4, 1, BF16>(l2, p, nb, l);
    case 64 * 16 + 2: return launch_block<4, 2, BF16>(l2, p, nb, l);
    default: return hipErrorInvalidValue;
  }
}

hipError_t dispatch(const Variant& v, int ns, int w, int pol, const Params& p, unsigned nb,
                    const Launch& l) {
  if (is_block_shape(ns)) {
    return v.bf16 ? dispatch_block<true>(ns, w, v.l2, p, nb, l)
                  : dispatch_block<false>(ns, w, v.l2, p, nb, l);
  }
  if (!v.bf16 && !v.multi) return by_ns<false, false>(ns, w, pol, v.l2, p, nb, l);
  if (!v.bf16 && v.multi) return by_ns<false, true>(ns, w, pol, v.l2, p, nb, l);
  if (v.bf16 && !v.multi) return by_ns<true, false>(ns, w, pol, v.l2, p, nb, l);
  return by_ns<true, true>(ns, w, pol, v.l2, p, nb, l);
}

bool shape_supported(const Variant& v, int T, int ns, int w, int pol) {
  if (is_block_shape(ns)) {
    // block kernel: T = 2..4, nontemporal state stream, <= 128 rows a block
    return T >= 2 && T <= kBlockMaxTokens && pol == kPolicyNtBoth &&
           (w == 1 || w == 2 || w == 4 || w == 8) && ns * w <= kDim;
  }
  const bool pow2 = (ns == 1 || ns == 2 || ns == 4 || ns == 8) &&
                    (w == 1 || w == 2 || w == 4 || w == 8);
  if (!pow2 || ns * w > 32) return false;
  if (v.bf16 || v.multi) return pol == kPolicyDefault || pol == kPolicyNtBoth;
  return pol >= kPolicyDefault && pol <= kPolicyNtLoad;
}

bool aligned(const void* p, uintptr_t a) {
  return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

// Launch shape for B*HV heads: (rows per lane group, waves per block), with
// nontemporal state loads and stores.  From rocprofv3 kernel-trace sweeps of
// every shape on MI355X, in steps rotating over >= 1 GiB of states, at
// 8..8192 heads (qk4_v8 B = 1..64, qk16_v32 B = 1..256, qk8_v32 B = 128),
// separately for an fp32 state at T = 1, T = 2 and T = 4 and for a bf16
// state.  Few heads want many small blocks (every CU busy); a few hundred
// heads want fewer waves with more rows each (4-8 rows per lane group, one
// wave per block: 6-14% faster there than 2 rows x 4 waves); large batches
// stream at ~6.5 TB/s with 2 rows x 4 waves at T = 1, while at T = 4 the
// per-token arithmetic is large enough that 4 rows per lane group (per-head
// work shared by more rows) wins.  Past 4096 heads (the launches whose
// workgroups are grouped by XCD) fewer waves a block measured faster
// (kernel-stamped sweep of every shape, qk16_v32: B=256 T=1 2 x 2 159.2 us
// against 2 x 4 160.6, B=512 317.3 against 323.1; B=256 T=4 4 x 1 171.0
// against 4 x 2 173.4; T=2 2 x 8 165.9 against 2 x 4 171.0; B=128 within
// 0.2%).
struct ShapeRow {
  long long max_heads;
  int ns;
  int waves;
};
constexpr ShapeRow kShapeFp32[] = {
    {16, 1, 1}, {64, 2, 2}, {256, 4, 1}, {384, 8, 1}, {4096, 2, 4}, {-1, 2, 2}};
constexpr ShapeRow kShapeT2[] = {
    {16, 1, 1}, {32, 1, 4}, {64, 2, 1}, {128, 2, 4}, {256, 4, 1}, {768, 8, 1}, {4096, 2, 4},
    {-1, 2, 8}};
constexpr ShapeRow kShapeT3Plus[] = {
    {16, 1, 1}, {32, 1, 4}, {64, 2, 1}, {256, 2, 2}, {384, 4, 1}, {768, 4, 2},
    {1536, 8, 1}, {4096, 4, 2}, {-1, 4, 1}};
constexpr ShapeRow kShapeBf16[] = {
    {16, 1, 2}, {32, 1, 4}, {64, 2, 4}, {128, 2, 2}, {256, 2, 1}, {384, 2, 4},
    {768, 4, 4}, {2048, 2, 4}, {-1, 4, 4}};
// A bf16 state at T >= 3 is VALU-bound from a few hundred heads on: more
// rows per lane group share each token's per-head work (kernel-stamped
// sweep of every shape, lazy decay: 256 heads 8.48 -> 7.68 us, 2048 heads
// 38.0 -> 33.0 us, 8192 heads 127.9 -> 117.3 us at T = 4).
constexpr ShapeRow kShapeBf16T3Plus[] = {
    {16, 1, 2}, {32, 1, 4}, {64, 2, 4}, {128, 2, 2}, {512, 4, 2}, {-1, 8, 1}};

template <size_t N>
void pick_row(const ShapeRow (&table)[N], long long heads, int* ns, int* waves) {
  for (const ShapeRow& r : table) {
    if (r.max_heads < 0 || heads <= r.max_heads) {
      *ns = r.ns;
      *waves = r.waves;
      return;
    }
  }
}

// Head counts at which the block kernel (rows_per_lane_group 16/32/64)
// runs T = 2..4 tokens, and its shape, from rocprofv3 kernel-trace sweeps at
// qk16_v32 B = 1..512 (steady regime) that launch every block shape and the
// token loop's shapes in turn, round after round, so that all of them run
// in the same GPU state, checked at large batches by back-to-back launches
// (which is how a model's layers run).  bf16 state: the block kernel is
// faster from B = 1 at T = 4 (4.18 against 4.52 us), from B = 2 at T = 3
// and from B = 4 at T = 2 (B=256 back to back: T = 4 89.5 against 116.0 us,
// T = 3 88.1 against 98.0 us, T = 2 86.2 against 87.5 us); (32, 2) is within
// 2% of the best shape from 1024 heads on.  fp32 state (the dots on
// v_mfma_f32_16x16x4_f32): faster at T = 4 from B = 4 to B = 64 (kernel
// trace: B=4 6.42 against 6.82 us, B=8 8.36 against 9.48, B=32 25.9
// against 26.8, B=64 49.3 against 52.4; back to back at B=64 47.1 against
// 48.7) and at T = 3 around B = 32 (24.9 against 26.2 us); the same time
// as the token loop from B = 128 on (B=256 T=4: 176.8 against 176.6 us)
// and slower at T = 2, where the token loop stays.
struct BlockRow {
  int T;                 // 0: any of 2..4
  bool bf16;             // the state's dtype
  long long min_heads;
  long long max_heads;   // -1: no limit
  int rows;
  int waves;
};
constexpr BlockRow kBlockRows[] = {
    // bf16 state
    {4, true, 1, 128, 32, 1},     {3, true, 33, 128, 32, 1},   {2, true, 65, 128, 32, 1},
    {0, true, 129, 256, 32, 4},   {0, true, 257, 512, 32, 2},  {0, true, 513, 1024, 64, 1},
    {0, true, 1025, -1, 32, 2},
    // fp32 state
    {4, false, 65, 128, 32, 1},   {4, false, 129, 256, 16, 2}, {4, false, 257, 2048, 32, 1},
    {3, false, 513, 1024, 32, 2},
};

void choose_shape(long long heads, bool bf16, int T, int* ns, int* waves, int* policy) {
  *policy = kPolicyNtBoth;
  for (const BlockRow& r : kBlockRows) {
    const bool t_ok = r.T == 0 ? (T >= 2 && T <= kBlockMaxTokens) : r.T == T;
    if (t_ok && r.bf16 == bf16 && heads >= r.min_heads &&
        (r.max_heads < 0 || heads <= r.max_heads)) {
      *ns = r.rows;
      *waves = r.waves;
      return;
    }
  }
  if (bf16 && T >= 3) {
    pick_row(kShapeBf16T3Plus, heads, ns, waves);
  } else if (bf16) {
    pick_row(kShapeBf16, heads, ns, waves);
  } else if (T >= 3) {
    pick_row(kShapeT3Plus, heads, ns, waves);
  } else if (T == 2) {
    pick_row(kShapeT2, heads, ns, waves);
  } else {
    pick_row(kShapeFp32, heads, ns, waves);
  }
}

// Every argument of one decode call, with the launch shape resolved.
struct StepArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* state;        // null: start from zeros
  const float* A_log;
  const void* a;
  const float* dt_bias;
  const void* b;
  float scale;
  void* output;
  void* new_state;
  int B, T, H, HV, K, V;
  int state_bf16;
  int use_qk_l2norm;
  int ns, waves, policy;
};

// Kernel variant of a call: the multi-token loop for T > 1, and also for a
// null state (it starts from zeros; the single-token kernel always reads one).
Variant variant_of(const StepArgs& s) {
  return Variant{s.use_qk_l2norm != 0, s.state_bf16 != 0, s.T > 1 || s.state == nullptr};
}

// Host-side validation of a call (no HIP call): sizes, launch shape, null
// and misaligned pointers, partial overlap of state and new_state.
hipError_t validate(const StepArgs& s) {
  if (s.B < 0 || s.T < 1 || s.H <= 0 || s.HV <= 0 || s.HV % s.H != 0) return hipErrorInvalidValue;
  if (s.H > 32767) return hipErrorInvalidValue;  // packed in 15 bits (and grid y)
  if (s.HV / s.H > 65535) return hipErrorInvalidValue;  // packed with H into 32 bits
  if (s.K != kDim || s.V != kDim) return hipErrorInvalidValue;
  if (s.state_bf16 != 0 && s.state_bf16 != 1) return hipErrorInvalidValue;
  const Variant var = variant_of(s);
  if (!shape_supported(var, s.T, s.ns, s.waves, s.policy)) return hipErrorInvalidValue;
  if (s.B == 0) return hipSuccess;
  if (!s.q || !s.k || !s.v || !s.A_log || !s.a || !s.dt_bias || !s.b || !s.output ||
      !s.new_state)
    return hipErrorInvalidValue;
  // 16-byte state row slices, 8- or 16-byte q/k slices, up to 16-byte v/out runs.
  if (!aligned(s.state, 16) || !aligned(s.new_state, 16) || !aligned(s.q, 16) ||
      !aligned(s.k, 16) || !aligned(s.v, 16) || !aligned(s.output, 16) ||
      !aligned(s.A_log, 4) || !aligned(s.dt_bias, 4) || !aligned(s.a, 2) || !aligned(s.b, 2))
    return hipErrorInvalidValue;
  const size_t elem = s.state_bf16 ? 2 : 4;
  const size_t state_bytes = static_cast<size_t>(s.B) * s.HV * kDim * kDim * elem;
  if (s.state != nullptr && s.new_state != s.state) {
    const uintptr_t s0 = reinterpret_cast<uintptr_t>(s.state);
    const uintptr_t d0 = reinterpret_cast<uintptr_t>(s.new_state);
    if (s0 < d0 + state_bytes && d0 < s0 + state_bytes)
      return hipErrorInvalidValue;  // partial overlap: only exact aliasing
  }
  const long long tiles = kDim / (rows_per_wave(s.ns) * s.waves);
  const long long max_blocks = (1LL << 31) / (64LL * s.waves);
  if (max_blocks / (tiles * s.HV) < 1) return hipErrorInvalidValue;
  return hipSuccess;
}

// The launches of a validated call on `stream`: one per group of at most
// 65535 sequences (grid z) whose work-items fit in 32 bits.
hipError_t launch(const StepArgs& s, hipStream_t stream, hipEvent_t start_event,
                  hipEvent_t stop_event) {
  if (s.B == 0) return hipSuccess;
  const Variant var = variant_of(s);
  const size_t elem = s.state_bf16 ? 2 : 4;
  const long long tiles = kDim / (rows_per_wave(s.ns) * s.waves);
  const long long max_blocks = (1LL << 31) / (64LL * s.waves);
  long long batches_per_launch = max_blocks / (tiles * s.HV);
  if (batches_per_launch > 65535) batches_per_launch = 65535;  // grid z limit

  Params p;
  p.A_log = s.A_log;
  p.dt_bias = s.dt_bias;
  p.scale = s.scale;
  p.T = s.T;
  p.H = s.H;
  p.HV = s.HV;
  p.ratio = s.HV / s.H;
  const long long T = s.T, H = s.H, HV = s.HV;
  for (long long b0 = 0; b0 < s.B; b0 += batches_per_launch) {
    const long long nb = (s.B - b0) < batches_per_launch ? (s.B - b0) : batches_per_launch;
    const long long bt0 = b0 * T;
    p.q = static_cast<const uint16_t*>(s.q) + bt0 * H * kDim;
    p.k = static_cast<const uint16_t*>(s.k) + bt0 * H * kDim;
    p.v = static_cast<const uint16_t*>(s.v) + bt0 * HV * kDim;
    p.state = s.state == nullptr
                  ? nullptr
                  : static_cast<const char*>(s.state) + b0 * HV * kDim * kDim * elem;
    p.a = static_cast<const uint16_t*>(s.a) + bt0 * HV;
    p.b = static_cast<const uint16_t*>(s.b) + bt0 * HV;
    p.out = static_cast<uint16_t*>(s.output) + bt0 * HV * kDim;
    p.new_state = static_cast<char*>(s.new_state) + b0 * HV * kDim * kDim * elem;
    // Start stamp on the first launch, stop stamp on the last.
    Launch l;
    l.stream = stream;
    l.start = b0 == 0 ? start_event : nullptr;
    l.stop = b0 + nb == s.B ? stop_event : nullptr;
    const hipError_t e = dispatch(var, s.ns, s.waves, s.policy, p, static_cast<unsigned>(nb), l);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

StepArgs make_args(const void* q, const void* k, const void* v, const void* state,
                   const float* A_log, const void* a, const float* dt_bias, const void* b,
                   float scale, void* output, void* new_state, int B, int T, int H, int HV,
                   int K, int V, int state_bf16, int use_qk_l2norm, int ns, int waves,
                   int policy) {
  return StepArgs{q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state, B, T, H,
                  HV, K, V, state_bf16, use_qk_l2norm, ns, waves, policy};
}

// The library's launch shape for a call (unchanged shape fields when B or
// HV is invalid: validation rejects the call).
void choose_args_shape(StepArgs& s) {
  if (s.B < 0 || s.HV <= 0) return;
  choose_shape(static_cast<long long>(s.B) * s.HV, s.state_bf16 != 0, s.T, &s.ns, &s.waves,
               &s.policy);
}

}  // namespace gdn

using namespace gdn;

extern "C" {

int gdn_decode_step(const void* q, const void* k, const void* v,
                    const float* state, const float* A_log, const void* a,
                    const float* dt_bias, const void* b, float scale,
                    void* output, float* new_state, int B, int H, int HV,
                    int K, int V, int use_qk_l2norm, void* hip_stream) {
  return gdn_decode_steps(q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state,
                          B, 1, H, HV, K, V, 0, use_qk_l2norm, hip_stream);
}

int gdn_decode_steps(const void* q, const void* k, const void* v, const void* state,
                     const float* A_log, const void* a, const float* dt_bias,
                     const void* b, float scale, void* output, void* new_state,
                     int B, int T, int H, int HV, int K, int V, int state_bf16,
                     int use_qk_l2norm, void* hip_stream) {
  StepArgs s = make_args(q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state, B, T,
                         H, HV, K, V, state_bf16, use_qk_l2norm, 0, 0, 0);
  choose_args_shape(s);
  hipError_t e = validate(s);
  if (e != hipSuccess) return e;
  return launch(s, static_cast<hipStream_t>(hip_stream), nullptr, nullptr);
}

int gdn_decode_step_shaped(const void* q, const void* k, const void* v,
                           const void* state, const float* A_log,
                           const void* a, const float* dt_bias, const void* b,
                           float scale, void* output, void* new_state, int B,
                           int T, int H, int HV, int K, int V, int state_bf16,
                           int use_qk_l2norm, int rows_per_lane_group,
                           int waves_per_block, int cache_policy,
                           void* start_event, void* stop_event, void* hip_stream) {
  const StepArgs s = make_args(q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state,
                               B, T, H, HV, K, V, state_bf16, use_qk_l2norm,
                               rows_per_lane_group, waves_per_block, cache_policy);
  hipError_t e = validate(s);
  if (e != hipSuccess) return e;
  return launch(s, static_cast<hipStream_t>(hip_stream), static_cast<hipEvent_t>(start_event),
                static_cast<hipEvent_t>(stop_event));
}

int gdn_decode_launch_shape(int B, int T, int HV, int state_bf16,
                            int* rows_per_lane_group, int* waves_per_block,
                            int* cache_policy, long long* num_blocks) {
  if (B < 0 || T < 1 || HV <= 0 || (state_bf16 != 0 && state_bf16 != 1) ||
      !rows_per_lane_group || !waves_per_block || !cache_policy || !num_blocks)
    return hipErrorInvalidValue;
  int ns = 0, waves = 0, policy = 0;
  choose_shape(static_cast<long long>(B) * HV, state_bf16 != 0, T, &ns, &waves, &policy);
  *rows_per_lane_group = ns;
  *waves_per_block = waves;
  *cache_policy = policy;
  *num_blocks = static_cast<long long>(B) * HV * (kDim / (rows_per_wave(ns) * waves));
  return hipSuccess;
}

int gdn_decode_step_stamped(const void* q, const void* k, const void* v, const float* state,
                            const float* A_log, const void* a, const float* dt_bias,
                            const void* b, float scale, void* output, float* new_state, int B,
                            int H, int HV, int K, int V, int use_qk_l2norm,
                            int rows_per_lane_group, int waves_per_block,
                            unsigned long long* stamps, long long stamp_capacity,
                            void* hip_stream) {
  StepArgs s = make_args(q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state, B, 1,
                         H, HV, K, V, 0, use_qk_l2norm, rows_per_lane_group, waves_per_block,
                         kPolicyNtBoth);
  hipError_t e = validate(s);
  if (e != hipSuccess) return e;
  if (state == nullptr || stamps == nullptr || B == 0 || B > 65535)
    return hipErrorInvalidValue;
  const int ns = rows_per_lane_group, w = waves_per_block;
  const long long tiles = kDim / (kLaneGroups * ns * w);
  const long long waves_total = static_cast<long long>(B) * HV * tiles * w;
  if (stamp_capacity < waves_total * kStampsPerWave) return hipErrorInvalidValue;
  const unsigned ratio = static_cast<unsigned>(HV / H);
  const dim3 grid(ratio * static_cast<unsigned>(tiles), static_cast<unsigned>(H),
                  static_cast<unsigned>(B));
  const unsigned h_ratio = static_cast<unsigned>(H) | (ratio << 16);
  const bool l2 = use_qk_l2norm != 0;
  const hipStream_t stream = static_cast<hipStream_t>(hip_stream);
  const int32_t* no_seqlens = nullptr;
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(64 * w), 0, stream, state,
                       static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
                       static_cast<const uint16_t*>(v), static_cast<const uint16_t*>(a),
                       static_cast<const uint16_t*>(b), h_ratio, 1, A_log, dt_bias,
                       static_cast<uint16_t*>(output), static_cast<void*>(new_state), scale,
                       no_seqlens, 0, stamps);
    return hipGetLastError();
  };
  // the single-token launch shapes of the library's table
  if (ns == 1 && w == 1) return l2 ? go(gdn_decode_k128_stamped<1, 1, true>)
                                   : go(gdn_decode_k128_stamped<1, 1, false>);
  if (ns == 2 && w == 2) return l2 ? go(gdn_decode_k128_stamped<2, 2, true>)
                                   : go(gdn_decode_k128_stamped<2, 2, false>);
  if (ns == 4 && w == 1) return l2 ? go(gdn_decode_k128_stamped<4, 1, true>)
                                   : go(gdn_decode_k128_stamped<4, 1, false>);
  if (ns == 8 && w == 1) return l2 ? go(gdn_decode_k128_stamped<8, 1, true>)
                                   : go(gdn_decode_k128_stamped<8, 1, false>);
  if (ns == 2 && w == 4) return l2 ? go(gdn_decode_k128_stamped<2, 4, true>)
                                   : go(gdn_decode_k128_stamped<2, 4, false>);
  return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------
// Bound steps and their HIP graph (B = 1 serving: launch overhead).
// ---------------------------------------------------------------------------

struct gdn_decode_plan {
  gdn::StepArgs args;
  int device;          // the device current at creation (the buffers' device)
};

struct gdn_decode_graph {
  hipGraphExec_t exec;
};

int gdn_decode_plan_create(const void* q, const void* k, const void* v, const void* state,
                           const float* A_log, const void* a, const float* dt_bias,
                           const void* b, float scale, void* output, void* new_state, int B,
                           int T, int H, int HV, int K, int V, int state_bf16,
                           int use_qk_l2norm, gdn_decode_plan** plan) {
  if (plan == nullptr) return hipErrorInvalidValue;
  *plan = nullptr;
  StepArgs s = make_args(q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state, B, T,
                         H, HV, K, V, state_bf16, use_qk_l2norm, 0, 0, 0);
  choose_args_shape(s);
  const hipError_t e = validate(s);
  if (e != hipSuccess) return e;
  int device = -1;                 // -1: no device (then runs switch none)
  if (hipGetDevice(&device) != hipSuccess) device = -1;
  gdn_decode_plan* p = new (std::nothrow) gdn_decode_plan{s, device};
  if (p == nullptr) return hipErrorOutOfMemory;
  *plan = p;
  return hipSuccess;
}

int gdn_decode_plan_run(const gdn_decode_plan* const* plans, int n, void* hip_stream) {
  if (n < 0 || (n > 0 && plans == nullptr)) return hipErrorInvalidValue;
  for (int i = 0; i < n; ++i)
    if (plans[i] == nullptr) return hipErrorInvalidValue;
  if (n == 0) return hipSuccess;
  // each launch goes to its plan's device, made current for it (and the
  // caller's current device restored after)
  int caller = -1;
  if (hipGetDevice(&caller) != hipSuccess) caller = -1;
  const hipStream_t stream = static_cast<hipStream_t>(hip_stream);
  int cur = caller;
  hipError_t e = hipSuccess;
  for (int i = 0; i < n && e == hipSuccess; ++i) {
    const int dev = plans[i]->device;
    if (dev >= 0 && dev != cur) {
      e = hipSetDevice(dev);
      if (e != hipSuccess) break;
      cur = dev;
    }
    e = launch(plans[i]->args, stream, nullptr, nullptr);
  }
  if (cur != caller && caller >= 0) {
    const hipError_t r = hipSetDevice(caller);
    if (e == hipSuccess) e = r;
  }
  return e;
}

void gdn_decode_plan_destroy(gdn_decode_plan* plan) { delete plan; }

int gdn_decode_graph_create(const gdn_decode_plan* const* plans, int n,
                            gdn_decode_graph** graph) {
  if (graph == nullptr) return hipErrorInvalidValue;
  *graph = nullptr;
  if (n < 1 || plans == nullptr) return hipErrorInvalidValue;
  for (int i = 0; i < n; ++i)
    if (plans[i] == nullptr) return hipErrorInvalidValue;
  // The launches are recorded from a private stream of the current device
  // (default priority) in capture mode; the graph is instantiated once.
  hipStream_t s = nullptr;
  hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
  if (e != hipSuccess) return e;
  e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
  hipError_t launch_error = hipSuccess;
  if (e == hipSuccess) {
    for (int i = 0; i < n && launch_error == hipSuccess; ++i)
      launch_error = launch(plans[i]->args, s, nullptr, nullptr);
    hipGraph_t g = nullptr;
    e = hipStreamEndCapture(s, &g);   // always ends the capture, also after a failed launch
    if (e == hipSuccess && launch_error != hipSuccess) e = launch_error;
    hipGraphExec_t exec = nullptr;
    if (e == hipSuccess) e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    if (g != nullptr) (void)hipGraphDestroy(g);
    if (e == hipSuccess) {
      *graph = new (std::nothrow) gdn_decode_graph{exec};
      if (*graph == nullptr) {
        (void)hipGraphExecDestroy(exec);
        e = hipErrorOutOfMemory;
      }
    }
  }
  const hipError_t d = hipStreamDestroy(s);
  if (e == hipSuccess && d != hipSuccess) {
    // a nonzero return never leaves a handle behind: the caller stores none
    gdn_decode_graph_destroy(*graph);
    *graph = nullptr;
  }
  return e != hipSuccess ? e : d;
}

int gdn_decode_graph_launch(const gdn_decode_graph* graph, void* hip_stream) {
  if (graph == nullptr) return hipErrorInvalidValue;
  return hipGraphLaunch(graph->exec, static_cast<hipStream_t>(hip_stream));
}

void gdn_decode_graph_destroy(gdn_decode_graph* graph) {
  if (graph == nullptr) return;
  (void)hipGraphExecDestroy(graph->exec);
  delete graph;
}

const char* gdn_decode_error_string(int code) {
  return hipGetErrorString(static_cast<hipError_t>(code));
}

int gdn_decode_abi_version(void) { return 6; }

}  // extern "C"
