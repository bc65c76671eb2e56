// Flash attention for gfx950, wave-pipelined: the kernel that runs D = 128 attention without a causal mask
// (the DiT path: int8 or 16-bit scores, 16-bit P V). Semantics as attention.hip's kernels, which follow the
// reference kernel kernels/attention.metal:70-394 (scores in log2 units, key masking at L, int8 scores scaled
// by qs_i * ks_j, P rounded to the value type, O divided by the row sum at the end).
#include "attention_common.h"

#include <algorithm>

namespace h3 {
namespace {
// ---------------------------------------------------------------------------------------------------------------
// Wave-pipelined kernel (D = 128, no causal mask; int8 or 16-bit scores): 4 waves per workgroup, one per SIMD
// (the workgroup's LDS keeps a second one off the CU), 64 query rows per wave (two 32-query MFMA tiles that
// share every K and V operand read), 256 per workgroup. A single wave overlaps its own MFMAs with its own
// independent VALU work almost completely on CDNA4 (measured: 4 MFMAs of 32 cycles beside 32 fp32 VALU
// instructions take the VALU time plus ~5 cycles per MFMA), so the softmax of key block j runs interleaved
// with the MFMAs of two other blocks, sub-tile by sub-tile: for key tile t (32 keys) and query tile u,
//     P V of block j-1 (8 MFMAs) | softmax of block j (16 scores per lane) | S of block j+1 (4 to 8 MFMAs)
// Each sub-tile's score registers are overwritten by block j+1 right after block j's softmax read them, and
// its P registers by block j right after block j-1's P V read them, so no register set is double-buffered.
// The running maximum is checked after the exponentials: a block whose per-lane row sum exceeds the limit
// (2^30 with bf16 P: scores up to ~30 log2 units above the reference maximum pass; 2^15 with f16 P, whose
// largest finite value is 65504; also inf or NaN) or that meets the first valid keys is recomputed in a rare
// branch from its K and scales (still in their LDS ring slots) with the exact block maximum, after O and l are
// rescaled. A reference maximum below the true one only scales P by a power of two: P keeps its relative
// rounding, and the fp32 O and l keep their range (a row's l stays below 2^30 per key block).
// Staging: LDS-direct buffer loads two blocks ahead into 4-deep rings; one barrier per key block.
// P V MFMA with the O accumulator in AGPRs. Written as assembly so that only O (and Q, an operand the score
// MFMAs read from AGPRs) lives in the accumulation registers: the score MFMAs are built with VGPR results
// (-amdgpu-mfma-vgpr-form) and feed the softmax's VALU directly, and the compiler keeps track of their hazards.
// Hazards it cannot see across this assembly: a VALU read or write of O after these MFMAs is preceded by
// o_fence(o), and the P operand (written by VALU) is always produced in an earlier key step, behind a barrier.
// The build checks the generated code for both (h3metal_amd/isa_check.py).
template <int VT>
__device__ __forceinline__ void mma_pv_acc(f32x16 &acc, i16x8 a, typename Vec8<VT>::type b) {
  if constexpr (VT == T_BF16) asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
  else asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
// Wait states between the last P V MFMA writing O and VALU access to O (a 16-pass XDL result needs 18). The
// accumulators are operands of the fence, so no access to them can be moved above it.
__device__ __forceinline__ void o_fence(f32x16 (&o)[2][4]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 4"
               : "+a"(o[0][0]), "+a"(o[0][1]), "+a"(o[0][2]), "+a"(o[0][3]), "+a"(o[1][0]), "+a"(o[1][1]),
                 "+a"(o[1][2]), "+a"(o[1][3]));
}
__device__ __forceinline__ void o_fence(f32x16 (&o)[3][4]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 4"
               : "+a"(o[0][0]), "+a"(o[0][1]), "+a"(o[0][2]), "+a"(o[0][3]), "+a"(o[1][0]), "+a"(o[1][1]),
                 "+a"(o[1][2]), "+a"(o[1][3]), "+a"(o[2][0]), "+a"(o[2][1]), "+a"(o[2][2]), "+a"(o[2][3]));
}

// First int8 score MFMA of a chain, accumulating onto the seed: the bits of 1/(2 pi) are an inline constant of
// the srcC operand (no registers, no moves). Assembly, because the builtin materialises the constant vector in
// registers. The next MFMA of the chain (a builtin of the same opcode) reads the result as its srcC, which the
// matrix unit forwards back to back; nothing else reads it (checked by h3metal_amd/isa_check.py).
__device__ __forceinline__ i32x16 mma_i8_seeded(i32x4 a, i32x4 b) {
  i32x16 d;
  asm volatile("v_mfma_i32_32x32x32_i8 %0, %1, %2, 0x3e22f983" : "=v"(d) : "a"(a), "a"(b));
  return d;
}

constexpr int NWV = 4;              // waves per workgroup
constexpr int NU = WAVE_NU;         // 32-query MFMA tiles per wave (sharing every K and V operand read)
constexpr int BQV = WAVE_BQ;        // query rows per workgroup
static_assert(BQV == NWV * 32 * NU, "32 NU query rows per wave");
constexpr int NRV = 4;              // ring depth (blocks)
// accepted growth of a row sum per key block: bf16 P (fp32's exponent range) and f16 P (largest finite 65504)
template <int VT>
constexpr float sum_limit() { return VT == T_F16 ? 0x1p15f : 0x1p30f; }
// int8 score accumulators start from the bits of the float 1/(2 pi) (an inline constant of the MFMA's C operand,
// so the seed costs no register): with |q . k| <= 128 * 127^2 < 2^21 the sum stays inside that float's binade
// [2^-3, 2^-2), whose ulp is 2^-26, so the accumulator's bits ARE the float SEED_F + s * 2^-26 and
// fma(bits, ks, -SEED_F * ks) = s * ks * 2^-26 replaces an int -> float conversion and a multiply (the 2^26 is
// folded into the query scale). The rounding of -SEED_F * ks adds at most ks * 2^-26 (one unit of s).
constexpr int SEED_I = 0x3E22F983;
constexpr float SEED_F = 0.15915494f;  // the float whose bits are SEED_I
constexpr float SEED_SCALE = 67108864.0f;  // 2^26
#ifdef WAVE_NO_SEED
constexpr bool SEEDED = false;
#else
constexpr bool SEEDED = true;
#endif

template <int QKT>
struct CfgW {
  static constexpr bool QK8 = QKT == T_I8;
  static constexpr int D = 128;
  static constexpr int ESZ = QK8 ? 1 : 2;
  static constexpr int RB = D * ESZ;   // bytes per K row
  static constexpr int NP = RB / 16;   // 16-byte pieces per K row
  static constexpr int NCH = NP / 2;   // score MFMAs per 32x32 tile
  static constexpr int KBYTES = BK * RB, VBYTES = BK * D * 2;
  static constexpr int KOFF = 0, VOFF = NRV * KBYTES, SOFF = VOFF + NRV * VBYTES;
  // int8: key scales ks, then the seed corrections -SEED_F * ks (made in LDS once per block by the waves)
  static constexpr int COFF = SOFF + (QK8 ? NRV * BK * 4 : 0);
  static constexpr int LDS = COFF + (QK8 ? NRV * BK * 4 : 0);
  static constexpr int KDMA = KBYTES / (NWV * 1024);  // 16-byte LDS-direct loads per wave and block
  static constexpr int VDMA = VBYTES / (NWV * 1024);
};

template <int QKT, int VT, int OT, bool DUMP>
__global__ __launch_bounds__(NWV * 64) __attribute__((amdgpu_waves_per_eu(1, 1)))
void attention_wave_kernel(const char *__restrict__ Q, const char *__restrict__ K, const char *__restrict__ V,
                           char *__restrict__ O, const float *__restrict__ qs, const float *__restrict__ ks,
                           int *__restrict__ dump, AttnParams p, int nqb, Split sp) {
  using C = CfgW<QKT>;
  constexpr int D = C::D;
  constexpr bool QK8 = C::QK8;
  using VT8 = typename Vec8<VT>::type;
  using VE = typename Vec8<VT>::elem;
  using VP2 = typename Vec8<VT>::pair;
  using SAcc = typename std::conditional<QK8, i32x16, f32x16>::type;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const unsigned lds0 = (unsigned)(size_t)(__attribute__((address_space(3))) char *)smem;

#ifdef WAVE_TIMING2
  // timing-only builds: shader-clock ticks at entry, at the first key step and after the last P V, and the real
  // time (100 MHz) at entry and after the last P V, written to the output's first bytes (no output is written)
  __builtin_amdgcn_sched_barrier(0);
  const unsigned long long t_entry = __builtin_amdgcn_s_memtime(), r_entry = __builtin_amdgcn_s_memrealtime();
  __builtin_amdgcn_sched_barrier(0);
  unsigned long long t_loop = 0;
#endif
  const int tid = threadIdx.x, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = blockIdx.x;
  int lid, unit = -1;
  bool rev = false;
  if (b < sp.nfull) {
    const int nb = sp.nfull;
    const int per = nb >> 3, rem = nb & 7, xcd = b & 7, loc = b >> 3;
    lid = (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + loc;
#ifndef WAVE_NO_REV
    // Every other round of an XCD's workgroups (one per CU) takes the key blocks in the order L-2, ..., 0, L-1:
    // it starts on the blocks the round before it read last, still in the XCD's L2 (a head's K and V outgrow it)
    rev = sp.rnd > 0 && ((loc / sp.rnd) & 1);
#endif
  } else {
    unit = b - sp.nfull;
    lid = sp.nfull + unit / sp.s;
  }
  const int h = lid / nqb, qb = lid - h * nqb;
  const int kvh = h / (p.H / p.KVH);
  // this lane's query rows: q0 + 32 u for the two query tiles u
  const int q0 = qb * BQV + w * (32 * NU) + l32;

  // Q operands (B of S^T = K Q^T), kept in registers: row q0 + 32 u, piece 2c + hl of each 32-byte chunk c
  i32x4 qreg[NU][C::NCH];
#pragma unroll
  for (int u = 0; u < NU; u++) {
    const int q = q0 + 32 * u;
    const bool ok = q < p.Lq;
    const char *qrow = Q + ((size_t)h * p.q_rows + (ok ? q : 0)) * C::RB;
#pragma unroll
    for (int c = 0; c < C::NCH; c++) {
      i32x4 v = *(const i32x4 *)(qrow + (2 * c + hl) * 16);
      qreg[u][c] = ok ? v : i32x4{0, 0, 0, 0};
      asm volatile("" : "+a"(qreg[u][c]));  // from here on Q lives in AGPRs only
    }
  }
  float qsc[NU];
#pragma unroll
  for (int u = 0; u < NU; u++) {
    const int q = q0 + 32 * u;
    qsc[u] = p.scale;
    if constexpr (QK8) qsc[u] = q < p.Lq ? fmaxf(qs[(size_t)h * p.q_rows + q] * p.scale, FLT_MIN) : 1.0f;
  }
  // the query scales of the main loop's seeded scores (s * ks * 2^-26)
  float qsw[NU];
#pragma unroll
  for (int u = 0; u < NU; u++) qsw[u] = QK8 && SEEDED ? qsc[u] * SEED_SCALE : qsc[u];

  int key0 = 0, Lk = p.L;
  if (unit >= 0) {
    key0 = (unit % sp.s) * sp.cb * BK;
    Lk = min(p.L, key0 + sp.cb * BK) - key0;
  }
  const char *Kh = K + ((size_t)kvh * p.k_rows + key0) * C::RB;
  const char *Vh = V + ((size_t)kvh * p.k_rows + key0) * D * 2;
  const float *ksh = QK8 ? ks + (size_t)kvh * p.k_rows + key0 : nullptr;
  const int nblk = Lk > 0 ? (Lk + BK - 1) / BK : 0;
  // the key block that step j works on; the partial block (if any) stays last, blocks past the end stay there
  auto kblk = [&](int j) { return __builtin_amdgcn_readfirstlane(rev && j < nblk - 1 ? nblk - 2 - j : j); };

  // -- LDS-direct staging. Load instruction r of this wave writes 1 KB at LDS (r * NWV + w) * 1024 of the block's
  // ring slot; each lane fetches the 16-byte piece whose swizzled position that is. One descriptor per array
  // covers this workgroup's Lk rows; the block's offset goes into the lane's VGPR offset (the part of the
  // address the range check covers), so rows at or past Lk, and blocks past the end, read as zero.
  auto rsrc = [&](const void *base, int row_bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0,
                                             __builtin_amdgcn_readfirstlane((int)((unsigned)max(0, Lk) * (unsigned)row_bytes)),
                                             0x00020000);
  };
  const __amdgpu_buffer_rsrc_t rk = rsrc(Kh, C::RB), rv = rsrc(Vh, D * 2);
  const __amdgpu_buffer_rsrc_t rs = QK8 ? rsrc(ksh, 4) : rk;
  unsigned kgo[C::KDMA], vgo[C::VDMA];
#pragma unroll
  for (int r = 0; r < C::KDMA; r++) {
    const int o = (r * NWV + w) * 1024 + 16 * lane;
    const int row = o / C::RB, slot = (o / 16) % C::NP;
    kgo[r] = row * C::RB + (slot ^ kswz<C::RB, C::NP>(row)) * 16;
  }
#pragma unroll
  for (int r = 0; r < C::VDMA; r++) {
    const int o = (r * NWV + w) * 1024 + 16 * lane;
    const int row = o >> 8, uu = (o & 255) >> 5, sub = (o >> 4) & 1;
    vgo[r] = row * (D * 2) + (2 * (uu ^ (2 * (row & 3))) + sub) * 16;
  }
  auto stage_k = [&](int blk) {  // K and key scales of block blk
    const int slot = blk & (NRV - 1);
    const unsigned kb0 = (unsigned)kblk(blk) * (BK * C::RB);
#pragma unroll
    for (int r = 0; r < C::KDMA; r++) dma16(lds0 + C::KOFF + slot * C::KBYTES + (r * NWV + w) * 1024, kgo[r] + kb0, rk);
    // every wave loads the block's 64 scales to the same place (no wave-dependent branch or wait count)
    if constexpr (QK8) dma4(lds0 + C::SOFF + slot * BK * 4, lane * 4 + (unsigned)kblk(blk) * (BK * 4), rs);
  };
  // the same loads one at a time (K and scales of block kb, V of block vb), so that they can be spread between
  // MFMAs: load i < KDMA is a K piece, then (int8) the scales, then the V pieces
  constexpr int NLOADS = C::KDMA + (QK8 ? 1 : 0) + C::VDMA;
  auto stage_one = [&](int i, int kb, int vb) {
    if (i < C::KDMA) {
      dma16(lds0 + C::KOFF + (kb & (NRV - 1)) * C::KBYTES + (i * NWV + w) * 1024,
            kgo[i] + (unsigned)kblk(kb) * (BK * C::RB), rk);
    } else if (QK8 && i == C::KDMA) {
      dma4(lds0 + C::SOFF + (kb & (NRV - 1)) * BK * 4, lane * 4 + (unsigned)kblk(kb) * (BK * 4), rs);
    } else {
      const int r = i - C::KDMA - (QK8 ? 1 : 0);
      dma16(lds0 + C::VOFF + (vb & (NRV - 1)) * C::VBYTES + (r * NWV + w) * 1024,
            vgo[r] + (unsigned)kblk(vb) * (BK * D * 2), rv);
    }
  };
  auto stage_v = [&](int blk) {
    const unsigned vb0 = (unsigned)kblk(blk) * (BK * D * 2);
#pragma unroll
    for (int r = 0; r < C::VDMA; r++)
      dma16(lds0 + C::VOFF + (blk & (NRV - 1)) * C::VBYTES + (r * NWV + w) * 1024, vgo[r] + vb0, rv);
  };

  f32x16 o[NU][D / 32];
#pragma unroll
  for (int u = 0; u < NU; u++)
#pragma unroll
    for (int db = 0; db < D / 32; db++)
#pragma unroll
      for (int i = 0; i < 16; i++) o[u][db][i] = 0.0f;
  // l: row sums up to the previous block; la: running partial row sums (four chains per query tile)
  float m[NU], l[NU];
  float nmv[NU];  // -m (0 while m = -inf): the exponent offset, changed only where m changes
  float la[NU][4];  // running partial row sums (four chains per query tile)
#pragma unroll
  for (int u = 0; u < NU; u++) {
    m[u] = -INFINITY;
    l[u] = nmv[u] = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; c++) la[u][c] = 0.0f;
  }
  SAcc s[2][NU];    // [key tile t][query tile u]
  i32x4 pb[2][NU][2]; // [t][u][16-key step within t]: 8 packed 16-bit P values (whole dwords, so that the
                     // rare path's writes merge with the common path's as whole registers)
#pragma unroll
  for (int t = 0; t < 2; t++)
#pragma unroll
    for (int u = 0; u < NU; u++) {
#pragma unroll
      for (int i = 0; i < 16; i++) s[t][u][i] = 0;
#pragma unroll
      for (int i = 0; i < 8; i++) pb[t][u][i >> 2][i & 3] = 0;
    }

  const int krow = 16 * (l32 >> 4) + 8 * ((l32 >> 2) & 1) + 4 * ((l32 >> 3) & 1) + (l32 & 3);
  const int l16 = lane & 15;
  const int tr_row = l16 >> 2, tr_col = (l16 & 3) * 8;
  unsigned vbase[D / 32], kbase[C::NCH];
  {
    const int k0 = 8 * hl + tr_row;
#pragma unroll
    for (int db = 0; db < D / 32; db++) vbase[db] = voff<D>(k0, (db * 32 + (l32 & 16)) / 8) + tr_col;
#pragma unroll
    for (int c = 0; c < C::NCH; c++) kbase[c] = krow * C::RB + (((2 * c + hl) ^ kswz<C::RB, C::NP>(krow)) * 16);
  }

  // K operands of key tile t of block j (A of S^T = K Q^T)
  auto kops = [&](int j, int t, i32x4 (&ka)[C::NCH]) {
    const char *Ks = smem + C::KOFF + (j & (NRV - 1)) * C::KBYTES + 32 * t * C::RB;
#pragma unroll
    for (int c = 0; c < C::NCH; c++) ka[c] = *(const i32x4 *)(Ks + kbase[c]);
  };
  auto score_mfmas = [&](SAcc &acc, const i32x4 (&ka)[C::NCH], int u, bool seeded) {
    SAcc seed;
#pragma unroll
    for (int i = 0; i < 16; i++) seed[i] = seeded ? SEED_I : 0;
#pragma unroll
    for (int c = 0; c < C::NCH; c++) {
      if constexpr (QK8 && SEEDED) {
        if (c == 0 && seeded) {
          acc = mma_i8_seeded(ka[0], qreg[u][0]);
          continue;
        }
      }
      acc = mma_qk<QKT>(ka[c], qreg[u][c], c == 0 ? seed : acc);
    }
  };
  // V operands of key tile t of block j: [16-key step][channel block]
  auto vops = [&](int j, int t, i16x8 (&va)[2][D / 32]) {
    const char *Vs = smem + C::VOFF + (j & (NRV - 1)) * C::VBYTES;
#pragma unroll
    for (int s2 = 0; s2 < 2; s2++) {
      const int koff = (32 * t + 16 * s2) * (D * 2);
#pragma unroll
      for (int db = 0; db < D / 32; db++) {
        const i16x4 lo = lds_tr16(Vs + vbase[db] + koff);
        const i16x4 hi = lds_tr16(Vs + vbase[db] + koff + 4 * (D * 2));
        va[s2][db] = i16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
    }
  };
  // key scales of key tile t of block j, for this lane's 16 keys
  auto kscales = [&](int j, int t, f32x4 (&k4)[2][2]) {
    const float *ksc = (const float *)(smem + C::SOFF) + (j & (NRV - 1)) * BK;
#pragma unroll
    for (int s8 = 0; s8 < 2; s8++)
#pragma unroll
      for (int hh = 0; hh < 2; hh++) k4[s8][hh] = *(const f32x4 *)(ksc + 32 * t + 16 * s8 + 8 * hl + 4 * hh);
  };
  // scores of sub-tile (t, u) of block j in log2 units before the query scale; keys >= Lk at -inf (MASK)
  auto to_x = [&](const SAcc &acc, const f32x4 (&k4)[2][2], int j, int t, bool mask) {
    f32x16 x;
    if constexpr (QK8) {
#pragma unroll
      for (int s8 = 0; s8 < 2; s8++)
#pragma unroll
        for (int hh = 0; hh < 2; hh++)
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const int i = 8 * s8 + 4 * hh + e;
            x[i] = (float)acc[i] * k4[s8][hh][e];
          }
    } else {
      x = acc;
    }
    if (mask) {
#pragma unroll
      for (int i = 0; i < 16; i++)
        if (kblk(j) * BK + 32 * t + 16 * (i >> 3) + 8 * hl + (i & 7) >= Lk) x[i] = -INFINITY;
    }
    return x;
  };
  auto exps = [&](const f32x16 &x, float qs_u, float nm, i32x4 (&pr)[2]) {
    float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i += 2) {
      const float p0 = __builtin_amdgcn_exp2f(fmaf(x[i], qs_u, nm));
      const float p1 = __builtin_amdgcn_exp2f(fmaf(x[i + 1], qs_u, nm));
      const VP2 pp = {(VE)p0, (VE)p1};
      pr[i >> 3][(i & 7) >> 1] = __builtin_bit_cast(int, pp);
      if (i & 2) acc1 = sum2<VT>(pp, acc1);
      else acc0 = sum2<VT>(pp, acc0);
    }
    return acc0 + acc1;
  };
  auto dump_scores = [&](const SAcc &acc, int j, int t, int u, bool seeded) {
    if constexpr (DUMP) {
      const int q = q0 + 32 * u;
      if (q < p.Lq) {
        // four consecutive keys at a time, taken out of the accumulator as vectors (element-wise extraction of
        // an MFMA result vector has been miscompiled into a splat of element 0)
        const i32x16 a = __builtin_bit_cast(i32x16, acc) - (seeded ? SEED_I : 0);
        const i32x4 g[4] = {__builtin_shufflevector(a, a, 0, 1, 2, 3), __builtin_shufflevector(a, a, 4, 5, 6, 7),
                            __builtin_shufflevector(a, a, 8, 9, 10, 11), __builtin_shufflevector(a, a, 12, 13, 14, 15)};
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int key = key0 + kblk(j) * BK + 32 * t + 16 * (r >> 1) + 8 * hl + 4 * (r & 1);
          int *dst = dump + ((size_t)h * p.Lq + q) * p.L + key;
          if (key + 4 <= key0 + Lk && (p.L & 3) == 0) {
            *(i32x4 *)dst = g[r];
          } else {
#pragma unroll
            for (int e = 0; e < 4; e++)
              if (key + e < key0 + Lk) dst[e] = g[r][e];
          }
        }
      }
    }
  };

  // Operands of one key tile (32 keys) of a step: V of block j - 1 (A of the P V MFMAs: [16-key step][channel
  // block]), K of block j + 1 (A of the score MFMAs) and the key scales of block j.
  struct Ops {
    i16x8 va[8];  // index 4 * s2 + db
    i32x4 ka[C::NCH];
    f32x4 k4[4];  // keys 32 t + 16 (g / 2) + 8 hl + 4 (g % 2) + e of score group g
    f32x4 c4[4];  // -SEED_F * k4 (int8), made in the query tile 0 sub-tile for both query tiles
  };
  auto vread = [&](int j, int t, int k) {  // V(j) operand k of key tile t
    const char *Vs = smem + C::VOFF + (j & (NRV - 1)) * C::VBYTES + (32 * t + 16 * (k >> 2)) * (D * 2) + vbase[k & 3];
    const i16x4 lo = lds_tr16(Vs);
    const i16x4 hi = lds_tr16(Vs + 4 * (D * 2));
    return i16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  };
  auto kread = [&](int j, int t, int c) {  // K(j) operand, chunk c of key tile t
    return *(const i32x4 *)(smem + C::KOFF + (j & (NRV - 1)) * C::KBYTES + 32 * t * C::RB + kbase[c]);
  };
  auto sread = [&](int j, int t, int g) {  // scales of K(j), score group g of key tile t
    return *(const f32x4 *)((const float *)(smem + C::SOFF) + (j & (NRV - 1)) * BK + 32 * t + 16 * (g >> 1) + 8 * hl +
                            4 * (g & 1));
  };
  auto load_ops = [&](Ops &op, int j, int t) {  // all operands of tile t of step j
#pragma unroll
    for (int g = 0; g < 4; g++)
      if constexpr (QK8) op.k4[g] = sread(j, t, g);
#pragma unroll
    for (int k = 0; k < 8; k++) op.va[k] = vread(j - 1, t, k);
#pragma unroll
    for (int c = 0; c < C::NCH; c++) op.ka[c] = kread(j + 1, t, c);
  };

  // One (key tile t, query tile u) sub-tile of step j, in issue order: the P V MFMAs of block j - 1 and the
  // score MFMAs of block j + 1 spread between short runs of independent VALU work (groups of 4 scores of block j
  // in flight at once; the matrix pipe accepts one MFMA per 32 cycles, and a lone wave stalls on back-to-back
  // MFMAs and on VALU results it needs too early). When `refresh`, each operand is replaced by the one of the
  // next tile (jn, tn) right after its last use here.
  auto sub_tile = [&](Ops &op, int j, int t, int u, bool has_pv, bool has_next, bool mask, bool refresh, int jn,
                      int tn, float (&la)[4], int st0 = 0, int stn = 0, int sj = 0) {
    dump_scores(s[t][u], j, t, u, QK8 && SEEDED);
    if constexpr (QK8 && SEEDED) {
      if (u == 0) {  // the seed corrections of this key tile, shared by both query tiles
#pragma unroll
        for (int g = 0; g < 4; g++)
          op.c4[g] = *(const f32x4 *)((const float *)(smem + C::COFF) + (j & (NRV - 1)) * BK + 32 * t + 16 * (g >> 1) +
                                      8 * hl + 4 * (g & 1));
      }
    }
    const float nm = nmv[u];
    float xv[16];
    int npv = 0, ns = 0;
    auto pv = [&]() {  // next P V MFMA of this sub-tile (the operand refresh also when there is none)
      const int k = npv++;
      if (has_pv) mma_pv_acc<VT>(o[u][k & 3], op.va[k], __builtin_bit_cast(VT8, pb[t][u][k >> 2]));
      if (refresh) op.va[k] = vread(jn - 1, tn, k);
      if (k < stn) stage_one(st0 + k, sj + 3, sj + 1);  // staging loads st0 .. st0 + stn - 1 of step sj
    };
    auto sm = [&]() {  // next score MFMA of this sub-tile
      const int c = ns++;
      SAcc seed;
#pragma unroll
      for (int i = 0; i < 16; i++) seed[i] = QK8 && SEEDED ? SEED_I : 0;
      if (has_next) {
        if constexpr (QK8 && SEEDED) {
          if (c == 0) s[t][u] = mma_i8_seeded(op.ka[0], qreg[u][0]);
          else s[t][u] = mma_qk<QKT>(op.ka[c], qreg[u][c], s[t][u]);
        } else {
          s[t][u] = mma_qk<QKT>(op.ka[c], qreg[u][c], c == 0 ? seed : s[t][u]);
        }
      }
      if (refresh) op.ka[c] = kread(jn + 1, tn, c);
    };
    // VALU stages on score group g (scores 4 g .. 4 g + 3)
    auto cv = [&](int g) {  // int8: the seeded accumulator's bits as a float; 16-bit: the fp32 score itself
      // (the whole vector is cast: element-wise casts of an MFMA result have been compiled into a splat)
      const f32x16 sf = __builtin_bit_cast(f32x16, s[t][u]);
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int i = 4 * g + e;
        if constexpr (QK8 && SEEDED) xv[i] = sf[i];
        else if constexpr (QK8) xv[i] = (float)s[t][u][i];
        else xv[i] = s[t][u][i];
      }
    };
    auto mu = [&](int g) {  // int8: s * ks * 2^-26; keys past Lk to -inf
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int i = 4 * g + e;
        if constexpr (QK8 && SEEDED) xv[i] = fmaf(xv[i], op.k4[g][e], op.c4[g][e]);
        else if constexpr (QK8) xv[i] *= op.k4[g][e];
        if (mask && kblk(j) * BK + 32 * t + 16 * (i >> 3) + 8 * hl + (i & 7) >= Lk) xv[i] = -INFINITY;
      }
      if (QK8 && refresh && u == NU - 1) op.k4[g] = sread(jn, tn, g);
    };
    auto fm = [&](int g) {
#pragma unroll
      for (int e = 0; e < 4; e++) xv[4 * g + e] = fmaf(xv[4 * g + e], qsw[u], nm);
    };
    auto ex = [&](int g) {
#pragma unroll
      for (int e = 0; e < 4; e++) xv[4 * g + e] = __builtin_amdgcn_exp2f(xv[4 * g + e]);
    };
    auto pk = [&](int g) {  // round to the value type, into the P operand, and sum the rounded values
#pragma unroll
      for (int e = 0; e < 4; e += 2) {
        const int i = 4 * g + e;
        const VP2 pp = {(VE)xv[i], (VE)xv[i + 1]};
        pb[t][u][i >> 3][(i & 7) >> 1] = __builtin_bit_cast(int, pp);
#ifndef WAVE_NO_SUM
        la[(g & 1) * 2 + (e >> 1)] = sum2<VT>(pp, la[(g & 1) * 2 + (e >> 1)]);
#endif
      }
    };
#define SB __builtin_amdgcn_sched_barrier(0)
    if constexpr (QK8) {
      // 8 P V, 4 score MFMAs; 16 scores x (cvt, mul, fma, exp) + 8 (pack, sum)
      pv(); cv(0); SB; cv(1); SB; pv(); mu(0); SB; cv(2); SB; pv(); mu(1); SB; fm(0); SB; pv(); cv(3); SB;
      mu(2); SB; pv(); fm(1); SB; ex(0); SB; pv(); mu(3); SB; fm(2); SB; pv(); ex(1); SB; sm(); fm(3); SB;
      pv(); ex(2); SB; sm(); pk(0); SB; ex(3); SB; sm(); pk(1); SB; pk(2); SB; sm(); pk(3); SB;
    } else {
      // 8 P V, 8 score MFMAs; 16 scores x (fma, exp) + 8 (pack, sum); mu() only masks here
      pv(); cv(0); cv(1); mu(0); mu(1); SB; pv(); fm(0); SB; pv(); fm(1); SB; pv(); cv(2); cv(3); mu(2); mu(3);
      ex(0); SB; pv(); fm(2); SB;
      pv(); ex(1); SB; pv(); fm(3); SB; pv(); ex(2); SB; sm(); pk(0); SB; sm(); ex(3); SB; sm(); pk(1); SB;
      sm(); SB; sm(); pk(2); SB; sm(); SB; sm(); pk(3); SB; sm(); SB;
    }
#undef SB
  };

  // Step j: P V of block j - 1, softmax of block j, scores of block j + 1. The barrier sits before the last
  // sub-tile: the loads issued after it (K and scales of block j + 3, V of block j + 1) land during the next
  // step, and the last sub-tile reads the first operands of the next step, all of which landed and were
  // published by that barrier. Ring slots (4 deep): K(j + 3) replaces K(j - 1), last read in step j - 1's
  // recompute; V(j + 1) replaces V(j - 3); scales(j + 3) replace scales(j - 1).
#ifdef WAVE_TIMING
  // timing-only builds: shader-clock ticks per phase of the step, written to the scores buffer at the end
  unsigned long long tph[7] = {0, 0, 0, 0, 0, 0, 0}, tlast = 0;
  auto tick = [&](int k) {
    const unsigned long long now = __builtin_amdgcn_s_memtime();
    if (k >= 0) tph[k] += now - tlast;
    tlast = now;
  };
#else
  auto tick = [](int) {};
#endif
  auto step = [&](Ops &op, int j, bool has_pv, bool has_next, bool mask) {
    tick(-1);
    // V of block j + 1 replaces V(j - 3), last read in step j - 2, before the previous barrier: with int8
    // scores its loads are spread over the first three sub-tiles (measured faster; with 16-bit scores, whose
    // sub-tiles read twice the K operands, slower). K and scales of block j + 3 replace those of block j - 1
    // (read up to step j - 1's recompute) and wait for this step's barrier.
    constexpr int KS = C::KDMA + (QK8 ? 1 : 0);  // K and scale loads come first in stage_one's order
    constexpr int VE0 = QK8 ? C::VDMA : 0;       // V loads issued before the barrier
    static_assert(C::VDMA == 4, "V loads per wave and step");
    // sub-tiles (t, u) in order; the barrier precedes the last one, (1, NU - 1). With int8 scores the V loads go
    // 2, 1, 1 into the first three sub-tiles.
    float tot[NU];
    bool bad = false;
    int st = KS;
#pragma unroll
    for (int idx = 0; idx < 2 * NU - 1; idx++) {
      const int t = idx / NU, u = idx % NU;
      const int n = QK8 ? (idx == 0 ? 2 : idx <= 2 ? 1 : 0) : 0;
      const bool last_u = u == NU - 1;
      sub_tile(op, j, t, u, has_pv, has_next, mask, last_u, t == 0 ? j : j + 1, t == 0 ? 1 : 0, la[u], st, n, j);
      st += n;
      tick(idx < 3 ? idx : 2);
      if (t == 1) {
        // block j's row sums are the growth of the running partial sums; query tile u's are complete here. A
        // sum above the limit (or NaN) means a score far above the reference maximum: the block is recomputed
        // below
        tot[u] = (la[u][0] + la[u][1]) + (la[u][2] + la[u][3]);
        bad = bad | !(tot[u] - l[u] <= sum_limit<VT>());
      }
    }
    // this wave's loads of the previous step (this step's V loads, the newest, may still be in flight)
    if constexpr (QK8) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    tick(6);
    __syncthreads();
    tick(3);
    // the scales of block j + 2 landed before this barrier: their seed corrections, published by the next one
    // (every wave writes the same 64 values)
    float kv = 0.0f;
    if constexpr (QK8 && SEEDED) kv = ((const float *)(smem + C::SOFF))[((j + 2) & (NRV - 1)) * BK + lane];
    sub_tile(op, j, 1, NU - 1, has_pv, has_next, mask, true, j + 1, 0, la[NU - 1], 0, KS + (C::VDMA - VE0), j);
    if constexpr (QK8 && SEEDED) ((float *)(smem + C::COFF))[((j + 2) & (NRV - 1)) * BK + lane] = kv * -SEED_F;
    tick(4);
    tot[NU - 1] = (la[NU - 1][0] + la[NU - 1][1]) + (la[NU - 1][2] + la[NU - 1][3]);
    bad = bad | !(tot[NU - 1] - l[NU - 1] <= sum_limit<VT>());
#ifdef WAVE_NO_CHECK
    bad = false;
#endif
    // rare: a score far above the reference maximum, or the first block (no maximum yet; it always holds
    // valid keys, so m is finite after it): recompute block j's P with the exact maximum
    if (__builtin_expect(j == 0 || __builtin_amdgcn_ballot_w64(bad) != 0, 0)) {
      o_fence(o);  // P V MFMAs of this step may still be writing O
#pragma unroll
      for (int u = 0; u < NU; u++) {
        // block j's scores of query tile u again (K and scales are still in their ring slots)
        f32x16 xs[2];
        float bmax = -INFINITY;
#pragma unroll
        for (int t = 0; t < 2; t++) {
          i32x4 ka[C::NCH];
          kops(j, t, ka);
          f32x4 k4[2][2];
          if constexpr (QK8) kscales(j, t, k4);
          SAcc acc;
          score_mfmas(acc, ka, u, false);
          xs[t] = to_x(acc, k4, j, t, mask);
#pragma unroll
          for (int i = 0; i < 16; i++) bmax = fmaxf(bmax, xs[t][i]);
        }
        const float pm = fmaxf(bmax, __shfl_xor(bmax, 32)) * qsc[u];
        const float mn = fmaxf(m[u], pm);
        const float f = (m[u] == -INFINITY || mn == -INFINITY) ? 1.0f : __builtin_amdgcn_exp2f(m[u] - mn);
        m[u] = mn;
        l[u] *= f;
#pragma unroll
        for (int db = 0; db < D / 32; db++)
#pragma unroll
          for (int i = 0; i < 16; i++) o[u][db][i] *= f;
        const float nm = mn == -INFINITY ? 0.0f : -mn;
        nmv[u] = nm;
        tot[u] = l[u] + (exps(xs[0], qsc[u], nm, pb[0][u]) + exps(xs[1], qsc[u], nm, pb[1][u]));
        la[u][0] = tot[u];
        la[u][1] = la[u][2] = la[u][3] = 0.0f;
      }
      asm volatile("s_nop 2" ::: "memory");  // VALU writes of O before the next MFMA reads it
    }
#pragma unroll
    for (int u = 0; u < NU; u++) l[u] = tot[u];
    tick(5);
  };

  if (nblk > 0) {
    stage_k(0);
    stage_k(1);
    stage_k(2);
    stage_v(0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if constexpr (QK8 && SEEDED) {  // seed corrections of blocks 0 and 1
#pragma unroll
      for (int b2 = 0; b2 < 2; b2++)
        ((float *)(smem + C::COFF))[b2 * BK + lane] = ((const float *)(smem + C::SOFF))[b2 * BK + lane] * -SEED_F;
      __syncthreads();
    }
    {
      i32x4 ka[C::NCH];
#pragma unroll
      for (int t = 0; t < 2; t++) {
        kops(0, t, ka);
#pragma unroll
        for (int u = 0; u < NU; u++) score_mfmas(s[t][u], ka, u, QK8 && SEEDED);
      }
    }
    Ops op;
    load_ops(op, 0, 0);
#ifdef WAVE_TIMING2
    __builtin_amdgcn_sched_barrier(0);
    t_loop = __builtin_amdgcn_s_memtime();
    __builtin_amdgcn_sched_barrier(0);
#endif
    // first block (no P V yet), the steady state (no masking: every key of the block is valid), the last block
    if (nblk == 1) step(op, 0, false, false, true);
    else step(op, 0, false, true, false);
    int j = 1;
    for (; j + 1 < nblk; j++) step(op, j, true, true, false);
    if (nblk > 1) step(op, nblk - 1, true, false, true);
    // P V of the last block (its tile-0 V operands were read by the last step)
#pragma unroll
    for (int t = 0; t < 2; t++) {
      if (t == 1) {
#pragma unroll
        for (int k = 0; k < 8; k++) op.va[k] = vread(nblk - 1, 1, k);
      }
#pragma unroll
      for (int u = 0; u < NU; u++)
#pragma unroll
        for (int k = 0; k < 8; k++) mma_pv_acc<VT>(o[u][k & 3], op.va[k], __builtin_bit_cast(VT8, pb[t][u][k >> 2]));
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // loads past the last block land before the exit
    o_fence(o);  // inside the branch: no copy of O may come between the last MFMA and the fence
  }

#ifdef WAVE_TIMING2
  {
    __builtin_amdgcn_sched_barrier(0);
    const unsigned long long t_end = __builtin_amdgcn_s_memtime(), r_end = __builtin_amdgcn_s_memrealtime();
    if (lane == 0) {
      long long *tp = (long long *)O + ((size_t)blockIdx.x * NWV + w) * 8;
      tp[0] = (long long)t_entry;
      tp[1] = (long long)t_loop;
      tp[2] = (long long)t_end;
      tp[3] = (long long)r_entry;
      tp[4] = (long long)r_end;
      tp[5] = blockIdx.x;
      tp[7] = nblk;
    }
    return;
  }
#endif
#ifdef WAVE_TIMING
  // the output's first bytes carry the ticks (workgroup b, wave w at 64 (NWV b + w)); no output is written
  if (lane == 0) {
    long long *tp = (long long *)O + ((size_t)blockIdx.x * NWV + w) * 8;
    for (int k = 0; k < 7; k++) tp[k] = (long long)tph[k];
    tp[7] = nblk;
  }
  return;
#endif
#pragma unroll
  for (int u = 0; u < NU; u++) {
    const int q = q0 + 32 * u;
    const float lt = l[u] + __shfl_xor(l[u], 32);
    if (unit >= 0) {
      float *wrow = sp.ws + ((size_t)unit * BQV + (q - qb * BQV)) * (D + 4);
#pragma unroll
      for (int db = 0; db < D / 32; db++)
#pragma unroll
        for (int g = 0; g < 4; g++)
          store4<T_F32>((char *)(wrow + db * 32 + 8 * g + 4 * hl), o[u][db][4 * g], o[u][db][4 * g + 1],
                        o[u][db][4 * g + 2], o[u][db][4 * g + 3]);
      if (hl == 0) {
        wrow[D] = m[u];
        wrow[D + 1] = lt;
      }
      continue;
    }
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    if (q < p.Lq) {
      constexpr int OSZ = OT == T_F32 ? 4 : 2;
      const int seq = h / p.seq_heads;
      char *orow = O + (((size_t)seq * p.seq_rows + q) * p.o_stride + (size_t)(h - seq * p.seq_heads) * D) * OSZ;
#pragma unroll
      for (int db = 0; db < D / 32; db++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const int d = db * 32 + 8 * g + 4 * hl;
          store4<OT>(orow + d * OSZ, o[u][db][4 * g] * inv, o[u][db][4 * g + 1] * inv, o[u][db][4 * g + 2] * inv,
                     o[u][db][4 * g + 3] * inv);
        }
    }
  }
}


}  // namespace

#ifndef WAVE_KERNEL_ONLY
int launch_attention_wave(int qkt, int vt, int ot, bool dump, const Exec &ex, const Arg *args, const AttnParams &p,
                          int nqb, const Split &sp, std::string *err) {
  auto run = [&](auto kern, int lds) -> int {
    static bool attr_set[2][4][4][2] = {};  // one per specialisation (qkt, vt, ot, dump)
    bool &set = attr_set[qkt == T_I8][vt][ot][dump];
    if (!set) {
      hipError_t e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
      if (e != hipSuccess) {
        *err = std::string("hipFuncSetAttribute: ") + hipGetErrorString(e);
        return -1;
      }
      set = true;
    }
    const long ntiles = (long)nqb * p.H;
    const long ngroups = sp.s ? (long)sp.nfull + (ntiles - sp.nfull) * sp.s : ntiles;
    hipLaunchKernelGGL(kern, dim3((unsigned)ngroups), dim3(NWV * 64), lds, ex.stream, args[0].ptr, args[1].ptr,
                       args[2].ptr, args[3].ptr, (const float *)args[5].ptr, (const float *)args[6].ptr,
                       dump ? (int *)args[7].ptr : nullptr,
                       p, nqb, sp);
    if (sp.s) {
      const int rows = (int)(ntiles - sp.nfull) * BQV;
      switch (ot) {
        case T_BF16:
          hipLaunchKernelGGL((attention_merge<128, T_BF16, BQV>), dim3((unsigned)(rows / 4)), dim3(256), 0, ex.stream,
                             sp.ws, args[3].ptr, p, nqb, sp.nfull, sp.s);
          break;
        case T_F16:
          hipLaunchKernelGGL((attention_merge<128, T_F16, BQV>), dim3((unsigned)(rows / 4)), dim3(256), 0, ex.stream,
                             sp.ws, args[3].ptr, p, nqb, sp.nfull, sp.s);
          break;
        default:
          hipLaunchKernelGGL((attention_merge<128, T_F32, BQV>), dim3((unsigned)(rows / 4)), dim3(256), 0, ex.stream,
                             sp.ws, args[3].ptr, p, nqb, sp.nfull, sp.s);
      }
    }
    return 0;
  };
  auto with_ot = [&](auto qk_c, auto v_c, auto d_c) -> int {
    constexpr int QKT = decltype(qk_c)::value, VT = decltype(v_c)::value;
    constexpr bool DUMP = decltype(d_c)::value;
    constexpr int LDS = CfgW<QKT>::LDS;
    switch (ot) {
      case T_BF16: return run(attention_wave_kernel<QKT, VT, T_BF16, DUMP>, LDS);
      case T_F16: return run(attention_wave_kernel<QKT, VT, T_F16, DUMP>, LDS);
      default: return run(attention_wave_kernel<QKT, VT, T_F32, DUMP>, LDS);
    }
  };
  using I8 = std::integral_constant<int, T_I8>;
  using B16 = std::integral_constant<int, T_BF16>;
  using F16 = std::integral_constant<int, T_F16>;
  auto with_dump = [&](auto qk_c, auto v_c) -> int {
    return dump ? with_ot(qk_c, v_c, std::true_type{}) : with_ot(qk_c, v_c, std::false_type{});
  };
  if (qkt == T_I8) return vt == T_BF16 ? with_dump(I8{}, B16{}) : with_dump(I8{}, F16{});
  if (qkt == T_BF16) return with_dump(B16{}, B16{});
  return with_dump(F16{}, F16{});
}
#endif

}  // namespace h3
