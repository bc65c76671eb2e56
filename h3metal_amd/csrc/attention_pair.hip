// Flash attention for gfx950 with two waves per SIMD: the kernel that runs int8-score attention at D = 128 without
// a causal mask (the DiT path's rotated int8 attention). Semantics as the other attention kernels, which follow the
// reference kernel kernels/attention.metal:70-394 (scores in log2 units, key masking at L, int8 scores scaled by
// qs_i * ks_j, P rounded to the value type, O divided by the row sum at the end).
//
// Structure. A workgroup is 8 waves (two per SIMD) over 256 query rows of one head: 4 pairs of waves, each pair
// owning 64 query rows (two 32-query MFMA tiles u = 0, 1). The two waves of a pair split the work of a 64-key block
// by role r (waves w and w + 4, r = w / 4):
//   * scores: wave r computes S^T = K Q^T for keys 32 r .. 32 r + 31 of the block and all 64 queries (8 int8
//     MFMAs, each K operand shared by both query tiles), and runs the softmax of those 2 x 32 x 32 scores;
//   * P V: wave r accumulates O for channels 64 r .. 64 r + 63 of all 64 queries over all 64 keys (16 bf16/f16
//     MFMAs), reading its own half of P from registers and its partner's half from LDS, where each wave leaves its
//     P of a block (4 KB) for the next step.
// Per wave that is half the register state of a one-wave-per-SIMD design with 64 rows (O 64 + Q 32 accumulation
// registers), so two waves fit one SIMD: one issues VALU work while the other's MFMAs run, which a single wave's
// instruction issue rate cannot do alone. The LDS operand traffic per CU is that of 64-row waves (each K and V
// operand read feeds two MFMAs), plus the P exchange.
//
// Running maximum: the pair shares one maximum per query row (both halves of P must be scaled alike). It is
// checked lazily after the exponentials (a block is accepted when every lane's row sum grew by at most the limit,
// i.e. no score far above the reference maximum; NaN and inf fail), and a block that fails anywhere in the
// workgroup, or the first block, is recomputed by every wave in a workgroup-uniform branch: each wave takes its
// half's exact block maximum, the pair exchanges the halves through LDS, both waves derive the same new maximum,
// rescale their O half and their partial row sums, and recompute their half of P. A reference maximum below the
// true one only scales P by a power of two, so the limit costs no precision.
//
// Pipeline of step j (one barrier per step): P V of block j - 1 | softmax of block j | scores of block j + 1,
// interleaved MFMA by MFMA with the VALU work in a fixed order (sched barriers). Staging: LDS-direct buffer loads
// (K, key scales of block j + 3 into 4-deep rings, V of block j + 1 into a 3-deep ring), waited for one step later.
#include "attention_common.h"

#include <algorithm>

namespace h3 {
namespace {

// P V MFMA with the O accumulator in AGPRs, as assembly (the score MFMAs are builtins with VGPR results that the
// softmax reads). Hazards the compiler cannot see across this assembly: a VALU access of O after these MFMAs is
// preceded by p_fence(o); P (written by VALU) is produced at least one MFMA earlier. The build checks the
// generated code for both (h3metal_amd/isa_check.py).
template <int VT>
__device__ __forceinline__ void pv_acc(f32x16 &acc, i16x8 a, i32x4 b) {
  if constexpr (VT == T_BF16) asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
  else asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
// 18 wait states between the last P V MFMA writing O and a VALU access of O; O is an operand so nothing moves above.
__device__ __forceinline__ void p_fence(f32x16 (&o)[2][2]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 4" : "+a"(o[0][0]), "+a"(o[0][1]), "+a"(o[1][0]), "+a"(o[1][1]));
}
// First int8 score MFMA of a chain onto the seed 1/(2 pi) (an inline constant of srcC); K from VGPRs, Q from AGPRs.
__device__ __forceinline__ i32x16 mma_i8_seed(i32x4 a, i32x4 b) {
  i32x16 d;
  asm volatile("v_mfma_i32_32x32x32_i8 %0, %1, %2, 0x3e22f983" : "=v"(d) : "v"(a), "a"(b));
  return d;
}

constexpr int NWP = 8;  // waves per workgroup (two per SIMD)
static_assert(PAIR_BQ == 256, "4 pairs of 64 query rows");
// int8 score accumulators start from the bits of the float 1/(2 pi): with |q . k| <= 128 * 127^2 < 2^21 the sum
// stays in that float's binade [2^-3, 2^-2), whose ulp is 2^-26, so the accumulator's bits ARE the float
// SEED_F + s * 2^-26, and fma(bits, ks, -SEED_F * ks) = s * ks * 2^-26 replaces an int -> float conversion and a
// multiply (2^26 is folded into the query scale).
constexpr int PSEED_I = 0x3E22F983;
constexpr float PSEED_F = 0.15915494f;
constexpr float PSEED_SCALE = 67108864.0f;  // 2^26
constexpr float PLIMIT_BF16 = 0x1p30f, PLIMIT_F16 = 0x1p15f;  // accepted row-sum growth per block (bf16 / f16 P)

struct CfgP {
  static constexpr int D = 128;
  static constexpr int RB = 128;  // bytes per K row (int8)
  static constexpr int NP = 8;    // 16-byte pieces per K row
  static constexpr int NCH = 4;   // score MFMAs per 32 x 32 tile (32 bytes of D each)
  static constexpr int NRK = 4, NRV = 3;  // ring depths: K and key scales, V
  static constexpr int KBYTES = BK * RB, VBYTES = BK * D * 2;
  static constexpr int KOFF = 0;
  static constexpr int VOFF = KOFF + NRK * KBYTES;
  static constexpr int SOFF = VOFF + NRV * VBYTES;
  static constexpr int POFF = SOFF + NRK * BK * 4;
  static constexpr int PBYTES = 4096;  // one wave's P of a block: [query tile][16-key step][lane] x 16 bytes
  static constexpr int FOFF = POFF + 2 * NWP * PBYTES;  // flags: [slot][wave] bytes
  static constexpr int XOFF = FOFF + 16;                // exchange of block maxima / row sums: [wave][u][32]
  static constexpr int LDS = XOFF + NWP * 2 * 32 * 4;
  static_assert(LDS <= 160 * 1024, "LDS of one CU");
  static_assert(KBYTES == NWP * 1024 && VBYTES == 2 * NWP * 1024, "one K and two V loads per wave and block");
};

// The body of the kernel for the waves of role R (0: waves 0-3, 1: waves 4-7). A function of its own per role, not
// inlined: the two roles run their steps in different orders, and one function holding both key loops exceeds the
// register file where each alone does not (each function has its own register allocation; the call is made once).
// Arguments reach the function in whatever registers the calling convention picks; these make them wave-uniform
// (scalar) again, which the buffer descriptors and the scalar address arithmetic need.
__device__ __forceinline__ int ufl(int x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ __forceinline__ float uff(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, x)));
}
template <class T>
__device__ __forceinline__ T *ufp(T *x) {
  const unsigned long long v = (unsigned long long)x;
  return (T *)(((unsigned long long)(unsigned)ufl((int)(v >> 32)) << 32) | (unsigned)ufl((int)v));
}

template <int VT, int OT, bool DUMP, int R>
__device__ __attribute__((noinline)) void pair_body(const char *Q_, const char *K_, const char *V_, char *O_,
                                                    const float *qs_, const float *ks_, int *dump_, AttnParams p_,
                                                    int nqb_, Split sp_) {
  const char *__restrict__ Q = ufp(Q_);
  const char *__restrict__ K = ufp(K_);
  const char *__restrict__ V = ufp(V_);
  char *__restrict__ O = ufp(O_);
  const float *__restrict__ qs = ufp(qs_);
  const float *__restrict__ ks = ufp(ks_);
  int *__restrict__ dump = ufp(dump_);
  const AttnParams p{ufl(p_.Lq), ufl(p_.L), ufl(p_.H), ufl(p_.KVH), ufl(p_.q_rows), ufl(p_.k_rows), ufl(p_.o_stride),
                     uff(p_.scale), ufl(p_.causal_off), ufl(p_.seq_heads), ufl(p_.seq_rows)};
  const int nqb = ufl(nqb_);
  const Split sp{ufl(sp_.nfull), ufl(sp_.s), ufl(sp_.cb), ufp(sp_.ws), ufl(sp_.rnd)};
  using C = CfgP;
  constexpr int D = C::D;
  using VE = typename Vec8<VT>::elem;
  using VP2 = typename Vec8<VT>::pair;
  constexpr float LIMIT = VT == T_F16 ? PLIMIT_F16 : PLIMIT_BF16;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const unsigned lds0 = (unsigned)(size_t)(__attribute__((address_space(3))) char *)smem;

  const int tid = threadIdx.x, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int pr = w & 3, wp = w ^ 4;  // pair, partner wave
  constexpr int r = R;              // role
  const int b = blockIdx.x;
  int lid, unit = -1;
  bool rev = false;
  if (b < sp.nfull) {
    // XCD-contiguous tile ranges (workgroup b runs on XCD b % 8)
    const int nb = sp.nfull;
    const int per = nb >> 3, rem = nb & 7, xcd = b & 7, loc = b >> 3;
    lid = (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + loc;
    // every other round of an XCD's workgroups takes the key blocks in the order L-2, ..., 0, L-1, starting on
    // the blocks the round before it read last (still in the XCD's L2)
    rev = sp.rnd > 0 && ((loc / sp.rnd) & 1);
  } else {
    unit = b - sp.nfull;
    lid = sp.nfull + unit / sp.s;
  }
  const int h = lid / nqb, qb = lid - h * nqb;
  const int kvh = h / (p.H / p.KVH);
  const int q0 = qb * PAIR_BQ + pr * 64 + l32;  // this lane's query rows: q0 + 32 u

  // Q operands (B of S^T = K Q^T) in AGPRs: row q0 + 32 u, piece 2 c + hl of each 32-byte chunk c
  i32x4 qreg[2][C::NCH];
#pragma unroll
  for (int u = 0; u < 2; u++) {
    const int q = q0 + 32 * u;
    const bool ok = q < p.Lq;
    const char *qrow = Q + ((size_t)h * p.q_rows + (ok ? q : 0)) * C::RB;
#pragma unroll
    for (int c = 0; c < C::NCH; c++) {
      i32x4 v = *(const i32x4 *)(qrow + (2 * c + hl) * 16);
      qreg[u][c] = ok ? v : i32x4{0, 0, 0, 0};
      asm volatile("" : "+a"(qreg[u][c]));
    }
  }
  float qsc[2], qsw[2];
#pragma unroll
  for (int u = 0; u < 2; u++) {
    const int q = q0 + 32 * u;
    qsc[u] = q < p.Lq ? fmaxf(qs[(size_t)h * p.q_rows + q] * p.scale, FLT_MIN) : 1.0f;
    qsw[u] = qsc[u] * PSEED_SCALE;
  }

  int key0 = 0, Lk = p.L;
  if (unit >= 0) {
    key0 = (unit % sp.s) * sp.cb * BK;
    Lk = min(p.L, key0 + sp.cb * BK) - key0;
  }
  const char *Kh = K + ((size_t)kvh * p.k_rows + key0) * C::RB;
  const char *Vh = V + ((size_t)kvh * p.k_rows + key0) * D * 2;
  const float *ksh = ks + (size_t)kvh * p.k_rows + key0;
  const int nblk = Lk > 0 ? (Lk + BK - 1) / BK : 0;
  auto kblk = [&](int j) { return __builtin_amdgcn_readfirstlane(rev && j < nblk - 1 ? nblk - 2 - j : j); };

  // -- LDS-direct staging: each wave loads 1 KB of K, 2 KB of V and (every wave, to the same place) the 64 key
  // scales of a block. One descriptor per array covers this workgroup's Lk rows; a block's offset goes into the
  // lane's VGPR offset (the range-checked part), so rows at or past Lk, and blocks past the end, read as zero.
  auto rsrc = [&](const void *base, int row_bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(
        (void *)base, (short)0, __builtin_amdgcn_readfirstlane((int)((unsigned)max(0, Lk) * (unsigned)row_bytes)),
        0x00020000);
  };
  const __amdgpu_buffer_rsrc_t rk = rsrc(Kh, C::RB), rv = rsrc(Vh, D * 2), rs = rsrc(ksh, 4);
  unsigned kgo, vgo[2];
  {
    const int o = w * 1024 + 16 * lane;
    const int row = o / C::RB, slot = (o / 16) % C::NP;
    kgo = row * C::RB + (slot ^ kswz<C::RB, C::NP>(row)) * 16;
#pragma unroll
    for (int rr = 0; rr < 2; rr++) {
      const int ov = (rr * NWP + w) * 1024 + 16 * lane;
      const int vrow = ov >> 8, uu = (ov & 255) >> 5, sub = (ov >> 4) & 1;
      vgo[rr] = vrow * (D * 2) + (2 * (uu ^ (2 * (vrow & 3))) + sub) * 16;
    }
  }
  // staging load i of the loads that fetch block kb's K and scales and block vb's V
  auto stage = [&](int i, int kb, int vb) {
    if (i == 0) {
      dma16(lds0 + C::KOFF + (kb % C::NRK) * C::KBYTES + w * 1024, kgo + (unsigned)kblk(kb) * C::KBYTES, rk);
    } else if (i == 1) {
      dma4(lds0 + C::SOFF + (kb % C::NRK) * BK * 4, lane * 4 + (unsigned)kblk(kb) * (BK * 4), rs);
    } else {
      const int rr = i - 2;
      dma16(lds0 + C::VOFF + (vb % C::NRV) * C::VBYTES + (rr * NWP + w) * 1024, vgo[rr] + (unsigned)kblk(vb) * C::VBYTES,
            rv);
    }
  };

  f32x16 o[2][2];  // [u][channel tile c]: channels 64 r + 32 c ..
#pragma unroll
  for (int u = 0; u < 2; u++)
#pragma unroll
    for (int c = 0; c < 2; c++)
#pragma unroll
      for (int i = 0; i < 16; i++) o[u][c][i] = 0.0f;
  float m[2], l[2], nmv[2], la[2][2];
#pragma unroll
  for (int u = 0; u < 2; u++) {
    m[u] = -INFINITY;
    l[u] = nmv[u] = 0.0f;
    la[u][0] = la[u][1] = 0.0f;
  }
  i32x16 s[2];      // [u] scores of this wave's key half
  i32x4 pb[2][2];   // [u][16-key step within the half] own P, packed 16-bit
#pragma unroll
  for (int u = 0; u < 2; u++) {
#pragma unroll
    for (int i = 0; i < 16; i++) s[u][i] = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) pb[u][i >> 2][i & 3] = 0;
  }

  // LDS addressing of the MFMA operands
  const int krow = 16 * (l32 >> 4) + 8 * ((l32 >> 2) & 1) + 4 * ((l32 >> 3) & 1) + (l32 & 3);
  const int l16 = lane & 15;
  const int tr_row = l16 >> 2, tr_col = (l16 & 3) * 8;
  unsigned vbase[2], kbase[C::NCH];
  {
    const int k0 = 8 * hl + tr_row;
#pragma unroll
    for (int c = 0; c < 2; c++) vbase[c] = voff<D>(k0, ((2 * r + c) * 32 + (l32 & 16)) / 8) + tr_col;
#pragma unroll
    for (int c = 0; c < C::NCH; c++)
      kbase[c] = 32 * r * C::RB + krow * C::RB + (((2 * c + hl) ^ kswz<C::RB, C::NP>(krow)) * 16);
  }
  auto vread = [&](int j, int st, int c) {  // V(j): keys 16 st .. 16 st + 15, channel tile 2 r + c (A of O^T = V^T P^T)
    const char *Vs = smem + C::VOFF + ((j + C::NRV) % C::NRV) * C::VBYTES + vbase[c] + 16 * st * (D * 2);
    const i16x4 lo = lds_tr16(Vs);
    const i16x4 hi = lds_tr16(Vs + 4 * (D * 2));
    return i16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  };
  auto kread = [&](int j, int c) {  // K(j), chunk c of this wave's key half
    return *(const i32x4 *)(smem + C::KOFF + (j % C::NRK) * C::KBYTES + kbase[c]);
  };
  auto sread = [&](int j, int g) {  // scales of K(j): keys 32 r + 16 (g / 2) + 8 hl + 4 (g % 2) + e
    return *(const f32x4 *)((const float *)(smem + C::SOFF) + (j % C::NRK) * BK + 32 * r + 16 * (g >> 1) + 8 * hl +
                            4 * (g & 1));
  };
  auto paddr = [&](int j, int wv, int u, int s2) {
    return C::POFF + ((((j + 2) & 1) * NWP + wv) * 4 + u * 2 + s2) * 1024 + lane * 16;
  };
  auto pwrite = [&](int j, int s2) {
#pragma unroll
    for (int u = 0; u < 2; u++) *(i32x4 *)(smem + paddr(j, w, u, s2)) = pb[u][s2];
  };
  auto pread = [&](int j, int u, int s2) { return *(const i32x4 *)(smem + paddr(j, wp, u, s2)); };
  auto dump_scores = [&](const i32x16 &acc, int j, int u, bool seeded) {
    if constexpr (DUMP) {
      const int q = q0 + 32 * u;
      if (q < p.Lq) {
        const i32x16 a = acc - (seeded ? PSEED_I : 0);
        const i32x4 g[4] = {__builtin_shufflevector(a, a, 0, 1, 2, 3), __builtin_shufflevector(a, a, 4, 5, 6, 7),
                            __builtin_shufflevector(a, a, 8, 9, 10, 11), __builtin_shufflevector(a, a, 12, 13, 14, 15)};
#pragma unroll
        for (int rr = 0; rr < 4; rr++) {
          const int key = key0 + kblk(j) * BK + 32 * r + 16 * (rr >> 1) + 8 * hl + 4 * (rr & 1);
          int *dst = dump + ((size_t)h * p.Lq + q) * p.L + key;
          if (key + 4 <= key0 + Lk && (p.L & 3) == 0) {
            *(i32x4 *)dst = g[rr];
          } else {
#pragma unroll
            for (int e = 0; e < 4; e++)
              if (key + e < key0 + Lk) dst[e] = g[rr][e];
          }
        }
      }
    }
  };
  auto exps = [&](const f32x16 &x, float qs_u, float nm, i32x4 (&pr2)[2]) {  // rare path: P and its row sum
    float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i += 2) {
      const float p0 = __builtin_amdgcn_exp2f(fmaf(x[i], qs_u, nm));
      const float p1 = __builtin_amdgcn_exp2f(fmaf(x[i + 1], qs_u, nm));
      const VP2 pp = {(VE)p0, (VE)p1};
      pr2[i >> 3][(i & 7) >> 1] = __builtin_bit_cast(int, pp);
      if (i & 2) acc1 = (acc1 + p0) + p1;
      else acc0 = (acc0 + p0) + p1;
    }
    return acc0 + acc1;
  };

  f32x4 k4[4];  // key scales of the block whose softmax runs next (prefetched at the end of the previous step)

  // Step j (0 <= j <= nblk): P V of block j - 1, softmax of block j, scores of block j + 1. One code path for every
  // step: the P V of block -1 reads zeroed LDS (V slot and the partners' P), the scores of blocks past the end are
  // those of zero K rows (the staging reads them as zero) and go unused, and step nblk only completes the P V of
  // the last block. Keys past Lk are masked in the exact path, which the last block always takes.
  auto step = [&](int j) {
    if constexpr (DUMP) {
      if (j < nblk) {
#pragma unroll
        for (int u = 0; u < 2; u++) dump_scores(s[u], j, u, true);
      }
    }
    float tot[2];
    // The two waves of a pair share a SIMD (waves w and w + 4) and run the step's three independent parts in
    // opposite orders, so that one is in its MFMA-heavy half (16 P V MFMAs) while the other is in its VALU-heavy
    // half (the softmax and the 8 score MFMAs). The wave in its softmax half runs at the higher priority: the
    // SIMD otherwise issues from the older wave first (role 0), which then finishes its step early and waits at
    // the barrier while role 1, fed only the leftover issue slots, catches up (measured with s_memtime: 2130 vs
    // 3130 ticks per step in the same code), and MFMAs, long and rarely issued, fill the softmax wave's gaps.
    auto seq = [&]() {
      // 16-key steps of the block in P V order: this wave's two, then its partner's
      constexpr int SS[4] = {2 * R, 2 * R + 1, 2 - 2 * R, 3 - 2 * R};
      i16x8 va[8];     // V(j - 1) operands, index 2 (position of the key step in SS) + channel tile
      i32x4 pp[2][2];  // partner's P(j - 1) [u][its 16-key step]
      i32x4 po[2][2];  // own P(j - 1) read back from LDS (role 1, whose softmax overwrites its P registers first)
      i32x4 ka[C::NCH];
      f32x4 c4[4];
      float xv[2][16];
      const f32x16 sf0 = __builtin_bit_cast(f32x16, s[0]), sf1 = __builtin_bit_cast(f32x16, s[1]);
      auto VR = [&](int n) { va[n] = vread(j - 1, SS[n >> 1], n & 1); };
      auto PR = [&](int u, int s2) { pp[u][s2] = pread(j - 1, u, s2); };
      auto PO = [&](int u, int s2) { po[u][s2] = *(const i32x4 *)(smem + paddr(j - 1, w, u, s2)); };
      auto KR = [&](int c) { ka[c] = kread(j + 1, c); };
      auto K4 = [&](int g) { k4[g] = sread(j + 1, g); };  // the next block's scales (after MU(g, *) of this one)
      auto PV = [&](int k) {  // k = 4 (position of the key step) + 2 c + u
        const int n = k >> 1, u = k & 1, ps = k >> 2;
        const i32x4 pop = ps == 0 ? (R == 0 ? pb[u][0] : po[u][0]) : ps == 1 ? (R == 0 ? pb[u][1] : po[u][1])
                        : ps == 2 ? pp[u][0] : pp[u][1];
        pv_acc<VT>(o[u][n & 1], va[n], pop);
      };
      auto SM = [&](int c, int u) {
        if (c == 0) s[u] = mma_i8_seed(ka[0], qreg[u][0]);
        else s[u] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ka[c], qreg[u][c], s[u], 0, 0, 0);
      };
      auto C4 = [&](int g) {
#pragma unroll
        for (int e = 0; e < 4; e++) c4[g][e] = k4[g][e] * -PSEED_F;
      };
      auto MU = [&](int g, int u) {  // s * ks * 2^-26 from the seeded bits
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int i = 4 * g + e;
          xv[u][i] = fmaf(u == 0 ? sf0[i] : sf1[i], k4[g][e], c4[g][e]);
        }
      };
      auto FM = [&](int g, int u) {
#pragma unroll
        for (int e = 0; e < 4; e++) xv[u][4 * g + e] = fmaf(xv[u][4 * g + e], qsw[u], nmv[u]);
      };
      auto EX = [&](int g, int u) {
#pragma unroll
        for (int e = 0; e < 4; e++) xv[u][4 * g + e] = __builtin_amdgcn_exp2f(xv[u][4 * g + e]);
      };
      auto PK = [&](int g, int u) {  // round to the value type into P; the row sums add the fp32 values (as nax.h:130 row_sum)
#pragma unroll
        for (int e = 0; e < 4; e += 2) {
          const int i = 4 * g + e;
          const VP2 v2 = {(VE)xv[u][i], (VE)xv[u][i + 1]};
          pb[u][i >> 3][(i & 7) >> 1] = __builtin_bit_cast(int, v2);
          la[u][e >> 1] = (la[u][e >> 1] + xv[u][i]) + xv[u][i + 1];
        }
      };
      // staging: K and scales of block j + 3, V of block j + 1
      auto ST = [&](int i) { stage(i, j + 3, j + 1); };
#define SB __builtin_amdgcn_sched_barrier(0)
      if constexpr (R == 0) {
        // P V of block j - 1 first (own P from registers), then the softmax of block j and the scores of j + 1
        __builtin_amdgcn_s_setprio(0);
        VR(0); VR(1); C4(0); C4(1); SB;
        PV(0); VR(2); ST(0); SB;
        PV(1); MU(0, 0); SB;
        PV(2); VR(3); SB;
        PV(3); MU(0, 1); ST(1); SB;
        PV(4); VR(4); PR(0, 0); PR(1, 0); SB;
        PV(5); MU(1, 0); SB;
        PV(6); VR(5); ST(2); SB;
        PV(7); MU(1, 1); SB;
        PV(8); VR(6); FM(0, 0); PR(0, 1); PR(1, 1); SB;
        PV(9); FM(0, 1); ST(3); SB;
        PV(10); VR(7); FM(1, 0); SB;
        PV(11); FM(1, 1); SB;
        PV(12); EX(0, 0); SB;
        PV(13); EX(0, 1); SB;
        PV(14); EX(1, 0); C4(2); C4(3); SB;
        PV(15); EX(1, 1); SB;
        __builtin_amdgcn_s_setprio(1);
        PK(0, 0); PK(0, 1); MU(2, 0); MU(2, 1); KR(0); KR(1); SB;
        PK(1, 0); PK(1, 1); MU(3, 0); MU(3, 1); pwrite(j, 0); KR(2); KR(3); SB;
        SM(0, 0); FM(2, 0); FM(2, 1); K4(0); K4(1); SB;
        SM(0, 1); FM(3, 0); FM(3, 1); K4(2); K4(3); SB;
        SM(1, 0); EX(2, 0); SB;
        SM(1, 1); EX(2, 1); SB;
        SM(2, 0); EX(3, 0); SB;
        SM(2, 1); EX(3, 1); SB;
        SM(3, 0); PK(2, 0); PK(2, 1); SB;
        SM(3, 1); PK(3, 0); PK(3, 1); pwrite(j, 1); SB;
      } else {
        // the softmax of block j and the scores of j + 1 first, then P V of block j - 1 (own P read back from LDS)
        __builtin_amdgcn_s_setprio(1);
        C4(0); C4(1); MU(0, 0); MU(0, 1); SB;
        MU(1, 0); MU(1, 1); FM(0, 0); FM(0, 1); ST(0); SB;
        FM(1, 0); FM(1, 1); EX(0, 0); EX(0, 1); KR(0); KR(1); SB;
        EX(1, 0); EX(1, 1); C4(2); C4(3); SB;
        PK(0, 0); PK(0, 1); MU(2, 0); MU(2, 1); KR(2); KR(3); SB;
        PK(1, 0); PK(1, 1); MU(3, 0); MU(3, 1); ST(1); SB;
        SM(0, 0); pwrite(j, 0); FM(2, 0); FM(2, 1); SB;
        SM(0, 1); FM(3, 0); FM(3, 1); SB;
        SM(1, 0); EX(2, 0); SB;
        SM(1, 1); EX(2, 1); ST(2); SB;
        SM(2, 0); EX(3, 0); VR(0); VR(1); SB;
        SM(2, 1); EX(3, 1); PO(0, 0); PO(1, 0); SB;
        SM(3, 0); PK(2, 0); PK(2, 1); VR(2); SB;
        SM(3, 1); PK(3, 0); PK(3, 1); pwrite(j, 1); ST(3); SB;
        __builtin_amdgcn_s_setprio(0);
        PV(0); VR(3); SB;
        PV(1); PO(0, 1); PO(1, 1); SB;
        PV(2); VR(4); SB;
        PV(3); SB;
        PV(4); VR(5); PR(0, 0); PR(1, 0); SB;
        PV(5); SB;
        PV(6); VR(6); SB;
        PV(7); SB;
        PV(8); VR(7); PR(0, 1); PR(1, 1); SB;
        PV(9); K4(0); K4(1); SB;
        PV(10); K4(2); K4(3); SB;
        PV(11); SB;
        PV(12); SB;
        PV(13); SB;
        PV(14); SB;
        PV(15); SB;
      }
#undef SB
    };
    seq();
    // block j's row sums (this wave's half) are the growth of the running partial sums; a sum above the limit (or
    // NaN) means a score far above the reference maximum somewhere in the block
    bool bad = false;
#pragma unroll
    for (int u = 0; u < 2; u++) {
      tot[u] = la[u][0] + la[u][1];
      bad = bad | !(tot[u] - l[u] <= LIMIT);
    }
    const bool mask = j == nblk - 1;
    const bool wbad = __builtin_amdgcn_ballot_w64(bad) != 0;
    if (lane == 0) *(unsigned char *)(smem + C::FOFF + (j & 1) * 8 + w) = wbad ? 1 : 0;
    // this wave's loads of the previous step have landed (this step's 4 may still be in flight)
    asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    __syncthreads();
    const unsigned long long flags = *(const unsigned long long *)(smem + C::FOFF + (j & 1) * 8);
    // rare (uniform over the workgroup): a score far above the reference maximum in some wave's half, or the
    // first block (no maximum yet): every wave recomputes its half of block j's P with the pair's exact maximum
    // (the last block, which holds the keys past Lk, always takes it: the common path does not mask)
    if (__builtin_expect(j < nblk && (j == 0 || mask || __builtin_amdgcn_readfirstlane((unsigned)(flags | (flags >> 32))) != 0), 0)) {
      p_fence(o);  // P V MFMAs of this step may still be writing O
      // block j's scores of this wave's half again (K and scales are still in their ring slots), in two passes
      // around the exchange of the halves' maxima (no score registers held across the barrier)
      auto rescore = [&](int u, auto &&use) {
        i32x16 acc;
#pragma unroll
        for (int i = 0; i < 16; i++) acc[i] = 0;
#pragma unroll
        for (int c = 0; c < C::NCH; c++) acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(kread(j, c), qreg[u][c], acc, 0, 0, 0);
        // keys at or past Lk: this lane's key 16 (i / 8) + (i % 8) of the half is key 32 r + 8 hl + that
        const int lim = mask ? Lk - kblk(j) * BK - 32 * r - 8 * hl : BK;
        asm volatile("" : "+v"(acc));  // one query tile's rescoring at a time
        f32x16 x;
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const f32x4 kk = sread(j, g);
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const int i = 4 * g + e;
            const float v = (float)acc[i] * kk[e];
            x[i] = 16 * (i >> 3) + (i & 7) >= lim ? -INFINITY : v;
          }
        }
        use(x);
      };
      float bm[2];
#pragma unroll
      for (int u = 0; u < 2; u++) {
        rescore(u, [&](const f32x16 &x) {
          float mx = -INFINITY;
#pragma unroll
          for (int i = 0; i < 16; i++) mx = fmaxf(mx, x[i]);
          bm[u] = fmaxf(mx, __shfl_xor(mx, 32));
        });
        if (hl == 0) ((float *)(smem + C::XOFF))[(w * 2 + u) * 32 + l32] = bm[u];
        __builtin_amdgcn_sched_barrier(0);
      }
      __syncthreads();
#pragma unroll
      for (int u = 0; u < 2; u++) {
        const float pm = fmaxf(bm[u], ((const float *)(smem + C::XOFF))[(wp * 2 + u) * 32 + l32]) * qsc[u];
        const float mn = fmaxf(m[u], pm);
        const float f = (m[u] == -INFINITY || mn == -INFINITY) ? 1.0f : __builtin_amdgcn_exp2f(m[u] - mn);
        m[u] = mn;
        l[u] *= f;
        // one 16-register tile at a time (the tiles live in AGPRs: a VALU multiply goes through VGPRs); the empty
        // volatile statements keep the compiler from batching the tiles' reads, which would need 64 VGPRs
#pragma unroll
        for (int c = 0; c < 2; c++) {
          f32x16 t = o[u][c];
          asm volatile("" : "+v"(t));
#pragma unroll
          for (int i = 0; i < 16; i++) t[i] *= f;
          asm volatile("" : "+v"(t));
          o[u][c] = t;
          asm volatile("" : "+a"(o[u][c]));
        }
        const float nm = mn == -INFINITY ? 0.0f : -mn;
        nmv[u] = nm;
        rescore(u, [&](const f32x16 &x) { tot[u] = l[u] + exps(x, qsc[u], nm, pb[u]); });
        __builtin_amdgcn_sched_barrier(0);
        la[u][0] = tot[u];
        la[u][1] = 0.0f;
      }
      pwrite(j, 0);
      pwrite(j, 1);
      __builtin_amdgcn_sched_barrier(0);
      // the scores and key scales of block j + 1 again (the common path computed them already): recomputing them
      // here keeps them out of this branch's live registers
#pragma unroll
      for (int u = 0; u < 2; u++) {
#pragma unroll
        for (int c = 0; c < C::NCH; c++) {
          const i32x4 kc = kread(j + 1, c);
          if (c == 0) s[u] = mma_i8_seed(kc, qreg[u][0]);
          else s[u] = __builtin_amdgcn_mfma_i32_32x32x32_i8(kc, qreg[u][c], s[u], 0, 0, 0);
        }
      }
#pragma unroll
      for (int g = 0; g < 4; g++) k4[g] = sread(j + 1, g);
      asm volatile("s_nop 2" ::: "memory");  // VALU writes of O before the next MFMA reads it
      __syncthreads();                       // the partner reads the recomputed P in the next step
    }
    if (j < nblk) {
#pragma unroll
      for (int u = 0; u < 2; u++) l[u] = tot[u];
    }
  };

  if (nblk > 0) {
    // the P V of block -1 (step 0) reads V ring slot 2 and P slot 1: zero them
#pragma unroll
    for (int i = 0; i < 2; i++)
      *(i32x4 *)(smem + C::VOFF + 2 * C::VBYTES + (i * NWP + w) * 1024 + lane * 16) = i32x4{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 4; i++) *(i32x4 *)(smem + C::POFF + ((NWP + w) * 4 + i) * 1024 + lane * 16) = i32x4{0, 0, 0, 0};
    stage(0, 0, 0); stage(1, 0, 0);
    stage(0, 1, 0); stage(1, 1, 0);
    stage(0, 2, 0); stage(1, 2, 0);
    stage(2, 0, 0); stage(3, 0, 0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 2; u++) {
#pragma unroll
      for (int c = 0; c < C::NCH; c++) {
        const i32x4 kc = kread(0, c);
        if (c == 0) s[u] = mma_i8_seed(kc, qreg[u][0]);
        else s[u] = __builtin_amdgcn_mfma_i32_32x32x32_i8(kc, qreg[u][c], s[u], 0, 0, 0);
      }
    }
#pragma unroll
    for (int g = 0; g < 4; g++) k4[g] = sread(0, g);
    for (int j = 0; j <= nblk; j++) step(j);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // loads past the last block land before the exit
    p_fence(o);
  }

  // row sums: this wave's half (two lanes per query), then the partner's through LDS
  float lt[2];
#pragma unroll
  for (int u = 0; u < 2; u++) {
    lt[u] = l[u] + __shfl_xor(l[u], 32);
    if (hl == 0) ((float *)(smem + C::XOFF))[(w * 2 + u) * 32 + l32] = lt[u];
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < 2; u++) lt[u] += ((const float *)(smem + C::XOFF))[(wp * 2 + u) * 32 + l32];

#pragma unroll
  for (int u = 0; u < 2; u++) {
    const int q = q0 + 32 * u;
    if (unit >= 0) {
      float *wrow = sp.ws + ((size_t)unit * PAIR_BQ + (q - qb * PAIR_BQ)) * (D + 4);
#pragma unroll
      for (int c = 0; c < 2; c++)
#pragma unroll
        for (int g = 0; g < 4; g++)
          store4<T_F32>((char *)(wrow + (2 * r + c) * 32 + 8 * g + 4 * hl), o[u][c][4 * g], o[u][c][4 * g + 1],
                        o[u][c][4 * g + 2], o[u][c][4 * g + 3]);
      if (hl == 0 && r == 0) {
        wrow[D] = m[u];
        wrow[D + 1] = lt[u];
      }
      continue;
    }
    const float inv = lt[u] > 0.0f ? 1.0f / lt[u] : 0.0f;
    if (q < p.Lq) {
      constexpr int OSZ = OT == T_F32 ? 4 : 2;
      const int seq = h / p.seq_heads;
      char *orow = O + (((size_t)seq * p.seq_rows + q) * p.o_stride + (size_t)(h - seq * p.seq_heads) * D) * OSZ;
#pragma unroll
      for (int c = 0; c < 2; c++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const int d = (2 * r + c) * 32 + 8 * g + 4 * hl;
          store4<OT>(orow + d * OSZ, o[u][c][4 * g] * inv, o[u][c][4 * g + 1] * inv, o[u][c][4 * g + 2] * inv,
                     o[u][c][4 * g + 3] * inv);
        }
    }
  }
}

template <int VT, int OT, bool DUMP>
__global__ __launch_bounds__(NWP * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attention_pair_kernel(const char *__restrict__ Q, const char *__restrict__ K, const char *__restrict__ V,
                           char *__restrict__ O, const float *__restrict__ qs, const float *__restrict__ ks,
                           int *__restrict__ dump, AttnParams p, int nqb, Split sp) {
  if (__builtin_amdgcn_readfirstlane(threadIdx.x >> 6) < 4) pair_body<VT, OT, DUMP, 0>(Q, K, V, O, qs, ks, dump, p, nqb, sp);
  else pair_body<VT, OT, DUMP, 1>(Q, K, V, O, qs, ks, dump, p, nqb, sp);
}

}  // namespace

int launch_attention_pair(int vt, int ot, bool dump, const Exec &ex, const Arg *args, const AttnParams &p, int nqb,
                          const Split &sp, std::string *err) {
  auto run = [&](auto kern) -> int {
    static bool attr_set[4][4][2] = {};
    bool &set = attr_set[vt][ot][dump];
    if (!set) {
      hipError_t e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, CfgP::LDS);
      if (e != hipSuccess) {
        *err = std::string("hipFuncSetAttribute: ") + hipGetErrorString(e);
        return -1;
      }
      set = true;
    }
    const long ntiles = (long)nqb * p.H;
    const long ngroups = sp.s ? (long)sp.nfull + (ntiles - sp.nfull) * sp.s : ntiles;
    hipLaunchKernelGGL(kern, dim3((unsigned)ngroups), dim3(NWP * 64), CfgP::LDS, ex.stream, args[0].ptr, args[1].ptr,
                       args[2].ptr, args[3].ptr, (const float *)args[5].ptr, (const float *)args[6].ptr,
                       dump ? (int *)args[7].ptr : nullptr, p, nqb, sp);
    if (sp.s) {
      const int rows = (int)(ntiles - sp.nfull) * PAIR_BQ;
      switch (ot) {
        case T_BF16:
          hipLaunchKernelGGL((attention_merge<128, T_BF16, PAIR_BQ>), dim3((unsigned)(rows / 4)), dim3(256), 0,
                             ex.stream, sp.ws, args[3].ptr, p, nqb, sp.nfull, sp.s);
          break;
        case T_F16:
          hipLaunchKernelGGL((attention_merge<128, T_F16, PAIR_BQ>), dim3((unsigned)(rows / 4)), dim3(256), 0,
                             ex.stream, sp.ws, args[3].ptr, p, nqb, sp.nfull, sp.s);
          break;
        default:
          hipLaunchKernelGGL((attention_merge<128, T_F32, PAIR_BQ>), dim3((unsigned)(rows / 4)), dim3(256), 0,
                             ex.stream, sp.ws, args[3].ptr, p, nqb, sp.nfull, sp.s);
      }
    }
    return 0;
  };
  auto with_ot = [&](auto v_c, auto d_c) -> int {
    constexpr int VT = decltype(v_c)::value;
    constexpr bool DUMP = decltype(d_c)::value;
    switch (ot) {
      case T_BF16: return run(attention_pair_kernel<VT, T_BF16, DUMP>);
      case T_F16: return run(attention_pair_kernel<VT, T_F16, DUMP>);
      default: return run(attention_pair_kernel<VT, T_F32, DUMP>);
    }
  };
  using B16 = std::integral_constant<int, T_BF16>;
  using F16 = std::integral_constant<int, T_F16>;
  if (vt == T_BF16) return dump ? with_ot(B16{}, std::true_type{}) : with_ot(B16{}, std::false_type{});
  return dump ? with_ot(F16{}, std::true_type{}) : with_ot(F16{}, std::false_type{});
}

}  // namespace h3
