// gdn_decode_block.h - device code of the block decode kernel: T = 2..4
// tokens per sequence applied to the state as one block, on the matrix cores
// (included by gdn_decode.hip).
//
// The token-by-token kernel (gdn_decode_kernel.h) spends three FMAs per state
// element per token (k.S, q.S and the rank-1 update) plus the dots' DPP
// reductions; at large batches and T >= 3 that VALU work, not HBM, sets its
// time.  Here every dot product is taken against the state S0 at the start
// of the step, as MFMA products, and the tokens' effects on each other are
// a small triangular recurrence per state row.  With raw (unnormalised)
// bf16 k_t, q_t, the decays g_t, Gamma_t = g_0 ... g_t, D(s,t) = g_{s+1} ...
// g_t, and per row (a 128-vector over k):
//
//   a_t = k_t . S0,  b_t = q_t . S0                      (MFMA, S0 read once)
//   x_t = kscale_t beta_t (v_t - kscale_t Gamma_t a_t
//                          - sum_{s<t} kscale_t D(s,t) (k_s . k_t) x_s)
//   o_t = qscale_t (Gamma_t b_t + sum_{s<=t} D(s,t) (k_s . q_t) x_s)
//   S_T = Gamma_{T-1} S0 + sum_s D(s,T-1) x_s k_s         (one MFMA per tile)
//
// x_t is kscale_t times the delta rule's d_t = beta_t (v_t - k_hat_t . g_t
// S_{t-1}) of token t (reference solution/triton/kernel.py:95-114 applied
// token after token, the recurrence of prefill_kernel.py:152-178), so S_t =
// g_t S_{t-1} + x_t k_t; expanding S_{t-1} in S0 and the earlier x_s gives
// the lines above.  No quantity is divided by a decay, so decays that
// underflow to zero need no special case.
//
// Lane layout (wave64, 16 x 16 MFMA tiles; lane = n + 16 g):
//   * a wave holds R tiles of 16 state rows; lane (n, g) holds row n of each
//     tile, at k = 32 s + 8 g + e for s, e = 0..7 (four 8-element runs,
//     16 contiguous bytes of a bf16 row, 32 of an fp32 row, per run);
//   * k.S and q.S: the state is the B operand (B[k][n] = S0[n][k]): for a
//     bf16 state the loaded bits as they are, of v_mfma_f32_16x16x32_bf16;
//     for an fp32 state each register as it is, of v_mfma_f32_16x16x4_f32
//     (32 products a tile, k = 32 s + 8 g + 4 h + i); row m of the A operand
//     is token m % 4's k (m & 4 clear) or q (m & 4 set), so lane n + 16 g
//     receives the dots of row n with the k's (g even) or the q's (g odd),
//     D[m][n] being in lane n + 16 (m / 4), register m % 4 (both products),
//     and a v_permlane16_swap gives every lane both;
//   * the update is v_mfma_f32_16x16x4_f32 per 16 x 16 tile of (k, row):
//     D[m][n] = C[m][n] + sum_t A[m][t] B[t][n], with C = Gamma S0 at the
//     lane's own elements, B[t][n] = D(t,T-1) x_t of row n from lane n + 16 t,
//     and A[m][t] = k_t at the tile's m-th k index from lane m + 16 t.  Tile
//     2 s + h covers k = 32 s + 8 g + 4 h + i (i = 0..3) in lane group g, so
//     its result registers are the lane's own run elements 4 h .. 4 h + 3:
//     the new state is stored from the registers the MFMA writes;
//   * A of the update comes from a product with a selector (a 32 x 16 0/1
//     matrix): k's A operand times the selector moves k_t[k(m)] to lane
//     m + 16 g, register t, exactly (bf16 values times 1.0).
// Per-head scalars (|k_t|^2, |q_t|^2, k_s.k_t, k_s.q_t) come from one more
// product of the k/q operand with itself, read with v_readlane.

#pragma once

#include "gdn_decode_kernel.h"

namespace gdn {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kBlockMaxTokens = 4;  // tokens per sequence the block kernel takes

__device__ __forceinline__ f32x4 mfma_bf16x32(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_f32x4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Register x[g] of a 4-vector, g the lane's group (a per-lane choice).
__device__ __forceinline__ float pick_by_group(f32x4 x, int g) {
  const float lo = g & 1 ? x[1] : x[0];
  const float hi = g & 1 ? x[3] : x[2];
  return g & 2 ? hi : lo;
}
__device__ __forceinline__ float pick_by_group(float x0, float x1, float x2, float x3, int g) {
  const float lo = g & 1 ? x1 : x0;
  const float hi = g & 1 ? x3 : x2;
  return g & 2 ? hi : lo;
}

typedef short s16x2 __attribute__((ext_vector_type(2)));

// A value the same in every lane, moved to a scalar register (VALU
// instructions take it as an operand; no vector register is held for it).
__device__ __forceinline__ float uniform(float x) {
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x)));
}

// Item e (0..7) of 8 packed bf16 values, as fp32.
__device__ __forceinline__ float bf16_item(u32x4 w, int e) {
  const uint32_t word = w[e >> 1];
  return e & 1 ? bf16_hi(word) : bf16_lo(word);
}

// Selector operand h (B of v_mfma_f32_16x16x32_bf16) of lane (n, g): item e
// is 1.0 where k index 8 g + e of the 32-long block is the tile's n-th,
// 8 (n / 4) + 4 h + n % 4.
__device__ __forceinline__ u32x4 selector(int n, int g, int h) {
  const int e = 4 * h + (n & 3);
  const uint32_t one = 0x3F80u << (16 * (e & 1));   // bf16 1.0 in the item's half
  const bool mine = g == (n >> 2);
  u32x4 r;
#pragma unroll
  for (int w = 0; w < 4; ++w) r[w] = (mine && (e >> 1) == w) ? one : 0u;
  return r;
}

// T = 2..4 tokens of R x 16 rows of one (b, hv) head per wave, WAVES waves
// per block; grid (ratio * tiles, H, B) as the token-by-token kernel's, with
// the same first eight (preloaded) arguments.  A null state starts from
// zeros.
// The new state leaves through LDS: the MFMA results give a lane 16 or 32
// bytes of a row at k = 32 s + 8 g, so a store straight from them writes 64
// bytes of each of 16 rows (half a 128-byte line) per instruction, which
// measured 1.34x the state's bytes in HBM writes (rocprofv3 WRITE_SIZE,
// B=256 T=4 bf16: 119.7 us) against 1.00x and 104.5 us through 16 padded
// LDS rows and whole-row stores; ordinary (write-back) stores from the
// registers also write 1.00x but took 117.5 us.  The R = 4 bf16 kernel is
// held to 168 VGPRs (3 waves per SIMD); held there too, the R = 2 fp32 one
// spills (B=64 T=4: 56 us against 49 us at 188 VGPRs, 2 waves per SIMD).
template <int R, int WAVES, bool L2NORM, bool BF16>
__global__ __launch_bounds__(64 * WAVES)
__attribute__((amdgpu_waves_per_eu((R == 4 && BF16) ? 3 : 1, 8)))
void gdn_decode_block(
    const void* state, const uint16_t* q, const uint16_t* k, const uint16_t* v,
    const uint16_t* a, const uint16_t* b, unsigned h_ratio, int T, const float* A_log_p,
    const float* dt_bias_p, uint16_t* out, void* new_state, float scale) {
  constexpr int kRowsPerWave = 16 * R;
  constexpr int kRowsPerBlock = kRowsPerWave * WAVES;
  constexpr int kTiles = kDim / kRowsPerBlock;
  static_assert(kDim % kRowsPerBlock == 0, "rows per block must divide 128");
  static_assert((kTiles & (kTiles - 1)) == 0, "tiles per head is a power of two");

  const int H = packed_heads(h_ratio);
  const int ratio = static_cast<int>(h_ratio >> 16);
  const int HV = H * ratio;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n = lane & 15;
  const int g = lane >> 4;

  const GridPos pos = decode_grid_pos<!BF16>(h_ratio);
  const int tile = pos.x & (kTiles - 1);
  const int hq = pos.y;
  const int bi = pos.z;
  const int hv = hq * ratio + pos.x / kTiles;
  const int head = bi * HV + hv;
  const int row0 = tile * kRowsPerBlock + wave * kRowsPerWave;
  const size_t tok0 = static_cast<size_t>(bi) * T;
  const bool has_state = state != nullptr;
  // LDS rows of one 16-row tile (the loaded state on its way into the MFMA
  // layout, then the new state on its way out), padded by 16 bytes so that
  // the 16 rows' accesses of one instruction spread over the banks
  constexpr int kRowBytes = kDim * (BF16 ? 2 : 4);
  constexpr int kPieces = kRowBytes / 16;           // 16-byte pieces a row
  constexpr int kLoads = 16 * kPieces / 64;         // 16-byte loads a lane per tile
  constexpr int kStageRow = kRowBytes + 16;
  constexpr int kStageBytes = 16 * kStageRow;
  __shared__ __attribute__((aligned(16))) char stage_mem[WAVES * kStageBytes];
  char* stage = stage_mem + wave * kStageBytes;

  // ---- loads: small inputs first, then the state -------------------------
  // k/q operand of lane (m, g): token m % 4 (zero past the last token), k
  // indices 32 s + 8 g .. + 7.
  const int tmc = (n & 3) < T ? (n & 3) : T - 1;
  u32x4 vk[4], vq[4];
  {
    const size_t base = ((tok0 + tmc) * H + hq) * kDim + 8 * g;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      vk[s] = *reinterpret_cast<const u32x4*>(k + base + 32 * s);
      vq[s] = *reinterpret_cast<const u32x4*>(q + base + 32 * s);
    }
  }
  // v of token t at each of the lane's rows (clamped token; a token past the
  // last one gets a zero coefficient below).
  // Two tokens' values share a register (halves of a 16-bit pair).
  s16x2 vbits[kBlockMaxTokens / 2][R];
#pragma unroll
  for (int tp = 0; tp < kBlockMaxTokens / 2; ++tp) {
    const int t0 = 2 * tp < T ? 2 * tp : T - 1;
    const int t1 = 2 * tp + 1 < T ? 2 * tp + 1 : T - 1;
    const size_t vb0 = ((tok0 + t0) * HV + hv) * kDim + row0 + n;
    const size_t vb1 = ((tok0 + t1) * HV + hv) * kDim + row0 + n;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      vbits[tp][r] = s16x2{static_cast<short>(v[vb0 + 16 * r]),
                           static_cast<short>(v[vb1 + 16 * r])};
    }
  }
  // gates of token min(lane, T - 1)
  const int tl = lane < T ? lane : T - 1;
  const uint16_t a_bits = a[(tok0 + tl) * HV + hv];
  const uint16_t b_bits = b[(tok0 + tl) * HV + hv];
  __builtin_amdgcn_sched_barrier(0);

  // The state loads are unconditional: a null state reads new_state (same
  // size, a valid address) and discards it below.  Loads that a branch may
  // skip would make the compiler's wait for the small inputs count as if
  // they had been skipped -- i.e. wait for the whole state first.
  // Whole rows: load i of tile r gives lane l 16 bytes, piece (64 i + l) % P
  // of row (64 i + l) / P (P pieces a row), so an instruction reads 1 KiB of
  // 4 (bf16) or 2 (fp32) whole rows; the tile is moved into the MFMA layout
  // through its LDS rows.  (Loaded directly in the MFMA layout, 64 bytes of
  // each of 16 rows an instruction, an in-place read-modify-write of 256 MiB
  // ran at half the bandwidth.)
  const size_t row_base = static_cast<size_t>(head) * kDim + row0;   // the wave's first row
  const char* src = static_cast<const char*>(has_state ? state
                                                       : static_cast<const void*>(new_state));
  u32x4 raw[R][kLoads];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int pc = i * 64 + lane;
      raw[r][i] = load_stream<u32x4, kPolicyNtBoth>(
          src + (row_base + 16 * r + pc / kPieces) * kRowBytes + (pc % kPieces) * 16);
    }
  __builtin_amdgcn_sched_barrier(0);
  const float A_log = A_log_p[hv];
  const float dt_bias = dt_bias_p[hv];
  __builtin_amdgcn_sched_barrier(0);

  // ---- per-head quantities (while the state is in flight) -----------------
  // Rows m % 4 >= T of the k/q operand hold token T-1's (finite) values:
  // every quantity they produce is multiplied by a zero coefficient (x_t = 0
  // for t >= T) or not stored.
  float gl, bl;
  gates(bf16_bits_to_f32(a_bits), dt_bias, A_log, bf16_bits_to_f32(b_bits), gl, bl);
  float gt[kBlockMaxTokens], bt[kBlockMaxTokens];
#pragma unroll
  for (int t = 0; t < kBlockMaxTokens; ++t) {
    gt[t] = lane_value(gl, t);
    bt[t] = lane_value(bl, t);
  }
  // Gram matrix of k_0..k_3 (rows 0-3) and q_0..q_3 (rows 4-7): lane j + 16 g,
  // register r holds vec_{4 g + r} . vec_j.
  // vn (rows m with m & 4 set: q_{m%4}, others k_{m%4}) is also the A
  // operand of the per-row dots: lane n + 16 g then receives k_t . S0 (g
  // even) or q_t . S0 (g odd) in register t.
  u32x4 vn[4];
  f32x4 gram = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    vn[s] = (n & 4) ? vq[s] : vk[s];
    gram = mfma_bf16x32(vn[s], vn[s], gram);
  }
  float kscale[kBlockMaxTokens], qscale[kBlockMaxTokens];
#pragma unroll
  for (int t = 0; t < kBlockMaxTokens; ++t) {
    if constexpr (L2NORM) {
      kscale[t] = __builtin_amdgcn_rsqf(lane_value(gram[t], t) + kL2Eps);
      qscale[t] = scale * __builtin_amdgcn_rsqf(lane_value(gram[t], 20 + t) + kL2Eps);
    } else {
      kscale[t] = 1.0f;
      qscale[t] = scale;
    }
  }
  // decays: Gamma_t, D(s,t) = g_{s+1} .. g_t; tokens past T - 1 count as no
  // decay in the final state's factors.
  float Gam[kBlockMaxTokens];
  Gam[0] = gt[0];
#pragma unroll
  for (int t = 1; t < kBlockMaxTokens; ++t) Gam[t] = Gam[t - 1] * gt[t];
  float gfin[kBlockMaxTokens];
#pragma unroll
  for (int t = 0; t < kBlockMaxTokens; ++t) gfin[t] = t < T ? gt[t] : 1.0f;
  float Dec[kBlockMaxTokens][kBlockMaxTokens];   // Dec[s][t], s <= t
#pragma unroll
  for (int s = 0; s < kBlockMaxTokens; ++s) {
    Dec[s][s] = 1.0f;
#pragma unroll
    for (int t = s + 1; t < kBlockMaxTokens; ++t) Dec[s][t] = Dec[s][t - 1] * gt[t];
  }
  float wc[kBlockMaxTokens];                      // D(s, T-1)
  wc[kBlockMaxTokens - 1] = 1.0f;
#pragma unroll
  for (int s = kBlockMaxTokens - 2; s >= 0; --s) wc[s] = wc[s + 1] * gfin[s + 1];
  const float gam_fin = uniform(gfin[0] * wc[0]);  // Gamma_{T-1}

  float ak[kBlockMaxTokens], bk[kBlockMaxTokens];
  float kc[kBlockMaxTokens][kBlockMaxTokens];     // kc[s][t], s < t
#pragma unroll
  for (int t = 0; t < kBlockMaxTokens; ++t) {
    ak[t] = uniform(kscale[t] * Gam[t]);
    bk[t] = uniform(t < T ? kscale[t] * bt[t] : 0.0f);
#pragma unroll
    for (int s = 0; s < t; ++s)
      kc[s][t] = uniform(kscale[t] * Dec[s][t] * lane_value(gram[s], t));
  }
  // this lane's output token g: o_g = my_aq b_g + sum_s my_qc[s] x_s
  float my_qc[kBlockMaxTokens];
  float my_aq;
  {
    float aq[kBlockMaxTokens];
    float qc[kBlockMaxTokens][kBlockMaxTokens];
#pragma unroll
    for (int t = 0; t < kBlockMaxTokens; ++t) {
      aq[t] = qscale[t] * Gam[t];
#pragma unroll
      for (int s = 0; s < kBlockMaxTokens; ++s)
        qc[s][t] = s <= t ? qscale[t] * Dec[s][t] * lane_value(gram[s], 4 + t) : 0.0f;
    }
    my_aq = pick_by_group(aq[0], aq[1], aq[2], aq[3], g);
#pragma unroll
    for (int s = 0; s < kBlockMaxTokens; ++s)
      my_qc[s] = pick_by_group(qc[s][0], qc[s][1], qc[s][2], qc[s][3], g);
  }
  const float my_wc = pick_by_group(wc[0], wc[1], wc[2], wc[3], g);

  // A operands of the update: tile 2 s + h, lane (m, g) = k_g at k index
  // 32 s + 8 (m / 4) + 4 h + m % 4.
  float ku[8];
  {
    const u32x4 sel0 = selector(n, g, 0);
    const u32x4 sel1 = selector(n, g, 1);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      ku[2 * s] = pick_by_group(mfma_bf16x32(vk[s], sel0, f32x4{0.0f, 0.0f, 0.0f, 0.0f}), g);
      ku[2 * s + 1] = pick_by_group(mfma_bf16x32(vk[s], sel1, f32x4{0.0f, 0.0f, 0.0f, 0.0f}), g);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  if (!has_state) {                    // uniform: start from zeros
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int i = 0; i < kLoads; ++i) raw[r][i] = u32x4{0u, 0u, 0u, 0u};
  }

  // ---- per tile of 16 rows: dots, recurrence, output, update --------------
#pragma unroll
  for (int r = 0; r < R; ++r) {
    // the tile into the MFMA layout: lane (n, g) gets row n at k = 32 s + 8 g
    // .. + 7 (bf16: one piece, 4 s + g; fp32: two, 8 s + 2 g + h)
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int pc = i * 64 + lane;
      *reinterpret_cast<u32x4*>(stage + (pc / kPieces) * kStageRow + (pc % kPieces) * 16) =
          raw[r][i];
    }
    __builtin_amdgcn_wave_barrier();
    u32x4 sb[4];          // bf16 state: the row's runs
    f32x4 sf[4][2];       // fp32 state
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if constexpr (BF16) {
        sb[s] = *reinterpret_cast<const u32x4*>(stage + n * kStageRow + 64 * s + 16 * g);
      } else {
#pragma unroll
        for (int h = 0; h < 2; ++h)
          sf[s][h] = *reinterpret_cast<const f32x4*>(stage + n * kStageRow + 128 * s + 32 * g +
                                                     16 * h);
      }
    }
    // k_t . S0 in the even lane groups, q_t . S0 in the odd ones; one swap of
    // odd and even groups (v_permlane16_swap) gives every lane both.
    f32x4 pn = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (BF16) {
#pragma unroll
      for (int s = 0; s < 4; ++s) pn = mfma_bf16x32(vn[s], sb[s], pn);
    } else {
      // fp32 state: v_mfma_f32_16x16x4_f32 with the contraction index k =
      // 32 s + 8 g + 4 h + i in lane group g, so the state registers are
      // the B operands as loaded and A is the k/q item at the same k (bf16
      // widened, exact); two accumulators halve the chain of dependent
      // products.
      f32x4 pn1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if (h == 0) pn = mfma_f32x4(bf16_item(vn[s], i), sf[s][0][i], pn);
            else pn1 = mfma_f32x4(bf16_item(vn[s], 4 + i), sf[s][1][i], pn1);
          }
      pn += pn1;
    }
    f32x4 pk, pq;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(pn[i]),
                                                       __float_as_uint(pn[i]), false, false);
      pk[i] = __uint_as_float(sw[0]);   // the even groups' values in every group
      pq[i] = __uint_as_float(sw[1]);   // the odd groups' values
    }
    float x[kBlockMaxTokens];
#pragma unroll
    for (int t = 0; t < kBlockMaxTokens; ++t) {
      const uint32_t vw = __builtin_bit_cast(uint32_t, vbits[t / 2][r]);
      const float vt = t & 1 ? bf16_hi(vw) : bf16_lo(vw);
      float acc = fmaf(-ak[t], pk[t], vt);
#pragma unroll
      for (int s = 0; s < t; ++s) acc = fmaf(-kc[s][t], x[s], acc);
      x[t] = bk[t] * acc;
    }
    float o = my_aq * pick_by_group(pq, g);
#pragma unroll
    for (int s = 0; s < kBlockMaxTokens; ++s) o = fmaf(my_qc[s], x[s], o);
    const float w = my_wc * pick_by_group(x[0], x[1], x[2], x[3], g);
    if (g < T) {
      out[((tok0 + g) * HV + hv) * kDim + row0 + 16 * r + n] =
          static_cast<uint16_t>(f32_to_bf16_bits(o));
    }
    if constexpr (BF16) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        f32x4 c0, c1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          c0[i] = gam_fin * bf16_item(sb[s], i);
          c1[i] = gam_fin * bf16_item(sb[s], 4 + i);
        }
        const f32x4 d0 = mfma_f32x4(ku[2 * s], w, c0);
        const f32x4 d1 = mfma_f32x4(ku[2 * s + 1], w, c1);
        const u32x4 packed{pack_bf16x2(d0[0], d0[1]), pack_bf16x2(d0[2], d0[3]),
                           pack_bf16x2(d1[0], d1[1]), pack_bf16x2(d1[2], d1[3])};
        *reinterpret_cast<u32x4*>(stage + n * kStageRow + 64 * s + 16 * g) = packed;
      }
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const f32x4 d = mfma_f32x4(ku[2 * s + h], w, gam_fin * sf[s][h]);
          *reinterpret_cast<f32x4*>(stage + n * kStageRow + 128 * s + 32 * g + 16 * h) = d;
        }
    }
    {
      // whole rows from the staging rows: 16 bytes a lane, 1 KiB an instruction
      __builtin_amdgcn_wave_barrier();
      constexpr int kLanesPerRow = kRowBytes / 16;          // 16 (bf16) or 32 (fp32)
      constexpr int kRowsPerStore = 64 / kLanesPerRow;     // 4 or 2
      const int lr = lane / kLanesPerRow;
      const int lc = lane % kLanesPerRow;
      char* dst = static_cast<char*>(new_state) + (static_cast<size_t>(head) * kDim + row0 + 16 * r) * kRowBytes;
#pragma unroll
      for (int i = 0; i < 16 / kRowsPerStore; ++i) {
        const int row = kRowsPerStore * i + lr;
        const u32x4 val = *reinterpret_cast<const u32x4*>(stage + row * kStageRow + 16 * lc);
        store_stream<u32x4, kPolicyNtBoth>(dst + row * kRowBytes + 16 * lc, val);
      }
      __builtin_amdgcn_wave_barrier();
    }
  }
}

}  // namespace gdn
