// Flash attention for gfx950 (CDNA4): out = softmax(scale * Q K^T) V per head,
// with int8 or 16-bit scores and 16-bit P V, online softmax in fp32.
//
// Semantics follow the reference kernel kernels/attention.metal:70-394:
//   Q [H][q_rows][D], K and V [KVH][k_rows][D], query head h reads key/value
//   head h / (H / KVH) (:87); keys >= L are masked, and with causal masking
//   query row i sees keys 0 .. i + causal_off (:115-117, :234-254); head h
//   writes rows (h / seq_heads) * seq_rows + i, columns (h % seq_heads) * D of
//   O (:384-385). With int8 scores (QK8) the score is
//   (q_i . k_j) * qs_i * ks_j * scale in log2 units (:101-106, :209-217), the
//   query scale applied in the exponent and the running maximum updated
//   lazily, only when a score exceeds it by SLACK = 8 (:255-298); P is rounded
//   to the value type before P V (:329-355); O is divided by the row sum at
//   the end (:376-393).
//
// The gfx950 design (not the Metal one):
//  * A workgroup is 8 waves in two groups of 4 (waves w and w + 4 share a SIMD).
//    Each wave owns 32 query rows of one head (256 per workgroup); the
//    workgroup walks the keys in blocks of BK = 64 staged in LDS.
//  * Ping-pong: every key block is two half-steps separated by workgroup
//    barriers. In a half-step one group runs its matrix phase (the score
//    MFMAs of block j and the P V MFMAs of block j-1) while the other group
//    runs its vector phase (the softmax of its block), then they swap. MFMA
//    and VALU work of the two waves on a SIMD overlap this way; a single
//    wave interleaving both does not overlap them well on CDNA4.
//  * Scores are computed transposed, S^T = K Q^T, on the 32x32 MFMA
//    (v_mfma_i32_32x32x32_i8 or v_mfma_f32_32x32x16_{bf16,f16}): an
//    accumulator lane holds 16 keys of ONE query (column = lane % 32), so the
//    softmax state (max, sum, rescale) is per lane; only the partner lane
//    (lane ^ 32, same query, other keys) is ever consulted.
//  * K rows of a 32-key tile are fed to the score MFMA in the order
//    pi(a) = 16*(a/16) + 8*((a/4)%2) + 4*((a/8)%2) + a%4, so that accumulator
//    element i of lane-half h holds key 16*(i/8) + 8*h + i%8: each half of the
//    accumulator is, as it stands, the B operand (8 consecutive keys per lane)
//    of one 32x32x16 P V MFMA computing O^T = V^T P^T, and O^T lands with the
//    same lane = query layout (rescaling O is a per-lane multiply).
//  * V stays row-major in LDS; its MFMA operand (4 keys x 1 channel per
//    read) comes from the transposing LDS read ds_read_b64_tr_b16: in each
//    16-lane group, source lane l addresses V[K0 + l/4][D0 + 4*(l%4) .. +3] and
//    destination lane i receives V[K0 .. K0+3][D0 + i]. V rows are swizzled in
//    32-byte units by key % 4 and K rows in 16-byte pieces by key bits 0, 1, 3,
//    so both LDS read patterns are bank-conflict free.
//  * Global loads are unconditional (rows clamped, out-of-range rows zeroed
//    after the load) so the compiler can count outstanding loads exactly;
//    the next block's loads are issued at the start of a key block and land in
//    LDS at the end of its second half-step.
//  * The 1-D grid is remapped so that each XCD (own L2) runs a contiguous
//    range of (head, query-block) tiles, which then share one head's K/V in L2.
//  * D = 128 without a causal mask (the DiT path) runs on the wave-pipelined
//    kernel of attention_wave.hip; this file's kernel serves every other case.
#include "attention_common.h"

#include <algorithm>
#include <cfloat>
#include <cmath>
#include <cstring>
#include <map>
#include <mutex>
#include <type_traits>

namespace h3 {
namespace {

constexpr int NW = 8;          // waves per workgroup (two groups of 4)
constexpr float SLACK = 8.0f;  // log2 units the running maximum may lag behind a score

template <int D, int QKT>
struct Cfg {
  static constexpr bool QK8 = QKT == T_I8;
  static constexpr int NT = NW * 64;             // threads
  static constexpr int BQ = NW * 32;             // query rows per workgroup
  static constexpr int ESZ = QK8 ? 1 : 2;        // bytes per Q/K element
  static constexpr int RB = D * ESZ;             // bytes per Q/K row
  static constexpr int NP = RB / 16;             // 16-byte pieces per Q/K row
  static constexpr int NCH = NP / 2;             // score MFMAs per 32x32 tile (one piece per lane half each)
  static constexpr int VP = D * 2 / 16;          // 16-byte pieces per V row
  static constexpr int KBYTES = BK * RB;
  static constexpr int VBYTES = BK * D * 2;
  static constexpr int KOFF = 0;                          // K ring: 2 blocks
  static constexpr int VOFF = 2 * KBYTES;                 // V ring: 2 blocks
  static constexpr int SOFF = VOFF + 2 * VBYTES;          // key-scale ring: 3 blocks
  static constexpr int LDS = QK8 ? SOFF + 3 * BK * 4 : SOFF;
  static_assert(D % 32 == 0 && D <= 128, "head dim");
};

// int8 scores: the int32 accumulators start at MAGIC, the bit pattern of the float 1.5 * 2^23. Adding a score
// s (|s| <= 128 * 127^2 < 2^22) keeps the sum in the binade [2^23, 2^24), where the float with those bits is
// exactly 1.5 * 2^23 + s. So s = float_bits(acc) - 1.5 * 2^23 exactly, a full-rate subtraction instead of a
// half-rate int->float conversion, and s * ks is one rounding. (Folding the subtraction into an fma with a
// per-key -1.5 * 2^23 * ks saves the subtraction but costs a second LDS vector per key, which measured slower.)
constexpr int MAGIC = 0x4B400000;
constexpr float MAGICF = 12582912.0f;


// DUMP: instead of attention, write the raw score accumulators S[h][q][key]
// (int32 for int8 inputs, fp32 otherwise) of the same MFMA path, for tests.
template <int DG, int QKT, int VT, int OT, bool CAUSAL, bool DUMP>
__global__ __launch_bounds__(NW * 64) void attention_kernel(const char *__restrict__ Q, const char *__restrict__ K,
                                                            const char *__restrict__ V, char *__restrict__ O,
                                                            const float *__restrict__ qs,
                                                            const float *__restrict__ ks, AttnParams p, int nqb,
                                                            Split sp) {
  // DG: the head dim of the tensors in memory; D: the head dim computed with (96 runs as 128: the missing
  // channels load as zeros, which changes no score and no output channel that is stored).
  constexpr int D = DG == 96 ? 128 : DG;
  using C = Cfg<D, QKT>;
  constexpr int RBG = DG * C::ESZ;  // bytes per Q/K row in memory
  using VT8 = typename Vec8<VT>::type;
  using VE = typename Vec8<VT>::elem;
  using VP2 = typename Vec8<VT>::pair;
  using SAcc = typename std::conditional<C::QK8, i32x16, f32x16>::type;
  extern __shared__ __attribute__((aligned(16))) char smem[];

  const int tid = threadIdx.x, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: keeps the group branches scalar
  const int grp = w >> 2;  // 0: matrix phase first in each key block, 1: vector phase first
  // XCD-aware tile order: workgroup b runs on XCD b % 8; give each XCD a contiguous range of the whole tiles.
  // Workgroups past them run one key chunk of a split tile each.
  const int b = blockIdx.x;
  int lid, unit = -1;
  if (b < sp.nfull) {
    const int nb = sp.nfull;
    const int per = nb >> 3, rem = nb & 7, xcd = b & 7, loc = b >> 3;
    lid = (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + loc;
  } else {
    unit = b - sp.nfull;
    lid = sp.nfull + unit / sp.s;
  }
  const int h = lid / nqb, qb = lid - h * nqb;
  const int kvh = h / (p.H / p.KVH);
  const int q = qb * C::BQ + w * 32 + l32;  // this lane's query row
  const bool qvalid = q < p.Lq;

  // Q operand (B of S^T = K Q^T): row q, piece 2c + hl of each 32-byte chunk c.
  i32x4 qreg[C::NCH];
  {
    const char *qrow = Q + ((size_t)h * p.q_rows + (qvalid ? q : 0)) * RBG;
#pragma unroll
    for (int c = 0; c < C::NCH; c++) {
      const int pc = 2 * c + hl;
      const bool in_row = pc * 16 < RBG;  // always true unless DG < D
      const i32x4 v = *(const i32x4 *)(qrow + (in_row ? pc : 0) * 16);
      qreg[c] = qvalid && in_row ? v : i32x4{0, 0, 0, 0};
    }
  }
  float qsc = p.scale;
  if constexpr (C::QK8) qsc = qvalid ? fmaxf(qs[(size_t)h * p.q_rows + q] * p.scale, FLT_MIN) : 1.0f;

  // keys of this workgroup: [key0, key0 + Lk) (a chunk of a split tile, or all L keys)
  int key0 = 0, Lk = p.L;
  if (unit >= 0) {
    key0 = (unit % sp.s) * sp.cb * BK;
    Lk = min(p.L, key0 + sp.cb * BK) - key0;
  }
  const char *Kh = K + ((size_t)kvh * p.k_rows + key0) * RBG;
  const char *Vh = V + ((size_t)kvh * p.k_rows + key0) * DG * 2;
  const float *ksh = C::QK8 ? ks + (size_t)kvh * p.k_rows + key0 : nullptr;
  int kend = Lk;
  if constexpr (CAUSAL) kend = min(p.L, qb * C::BQ + C::BQ + p.causal_off);  // never split
  const int nblk = kend > 0 ? (kend + BK - 1) / BK : 0;

  // -- staging: global -> registers -> LDS. Group g stages rows 32 g .. 32 g + 31 of every block. Buffer loads
  // with a per-block descriptor whose range ends at key L: rows at or beyond L read as zero (their keys are
  // masked, and their values must not turn 0 * garbage into NaN) and nothing past L is ever read. Offsets within
  // a block are per-thread constants; the descriptor's base advances in scalar registers.
  constexpr int HK = BK / 2;                       // rows staged per group
  constexpr int GT = C::NT / 2;                    // threads per group
  constexpr int KPT = (HK * C::NP + GT - 1) / GT;  // K pieces per thread
  constexpr int VPT = (HK * C::VP + GT - 1) / GT;  // V pieces per thread
  const int gt = tid & (GT - 1), row0 = grp * HK;
  i32x4 kr[KPT];
  i32x4 vr[VPT];
  float ksr = 0.0f;
  auto rsrc = [&](const void *base, int blk, int row_bytes) {
    const int rows = max(0, Lk - blk * BK);
    return __builtin_amdgcn_make_buffer_rsrc((void *)((const char *)base + (size_t)blk * BK * row_bytes), (short)0,
                                             rows * row_bytes, 0x00020000);
  };
  auto load_k = [&](int blk) {
    const __amdgpu_buffer_rsrc_t r = rsrc(Kh, blk, RBG);
#pragma unroll
    for (int i = 0; i < KPT; i++) {
      const int idx = (gt + i * GT) % (HK * C::NP);
      // pieces past a row in memory (DG < D) are sent out of the descriptor's range: they read as zero
      const int pc = idx % C::NP;
      const unsigned off = pc * 16 < RBG ? (row0 + idx / C::NP) * RBG + pc * 16 : 0x80000000u;
      kr[i] = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    }
    if constexpr (C::QK8)
      ksr = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc(ksh, blk, 4), (row0 + (gt & (HK - 1))) * 4, 0, 0));
  };
  auto load_v = [&](int blk) {
    const __amdgpu_buffer_rsrc_t r = rsrc(Vh, blk, DG * 2);
#pragma unroll
    for (int i = 0; i < VPT; i++) {
      const int idx = (gt + i * GT) % (HK * C::VP);
      const int pc = idx % C::VP;
      const unsigned off = pc * 16 < DG * 2 ? (row0 + idx / C::VP) * DG * 2 + pc * 16 : 0x80000000u;
      vr[i] = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    }
  };
  auto store_k = [&](int blk) {
    char *kbuf = smem + C::KOFF + (blk & 1) * C::KBYTES;
#pragma unroll
    for (int i = 0; i < KPT; i++) {
      const int idx = gt + i * GT;
      const int key = row0 + idx / C::NP, pc = idx % C::NP;
      if (idx < HK * C::NP) *(i32x4 *)(kbuf + key * C::RB + ((pc ^ kswz<C::RB, C::NP>(key)) * 16)) = kr[i];
    }
    if constexpr (C::QK8) {
      if (gt < HK) {
        ((float *)(smem + C::SOFF))[(blk % 3) * BK + row0 + gt] = ksr;
      }
    }
  };
  auto store_v = [&](int blk) {
    char *vbuf = smem + C::VOFF + (blk & 1) * C::VBYTES;
#pragma unroll
    for (int i = 0; i < VPT; i++) {
      const int idx = gt + i * GT;
      const int key = row0 + idx / C::VP, pc = idx % C::VP;
      if (idx < HK * C::VP) *(i32x4 *)(vbuf + voff<D>(key, pc)) = vr[i];
    }
  };

  f32x16 o[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; db++)
#pragma unroll
    for (int i = 0; i < 16; i++) o[db][i] = 0.0f;
  float m = -INFINITY, l = 0.0f;
  SAcc s[2];
  VT8 pb[2][2];
  SAcc sinit;
#pragma unroll
  for (int i = 0; i < 16; i++) sinit[i] = C::QK8 ? MAGIC : 0;
#pragma unroll
  for (int t = 0; t < 2; t++)
#pragma unroll
    for (int i = 0; i < 16; i++) {
      s[t][i] = 0;
      pb[t][i >> 3][i & 7] = (VE)0.0f;
    }

  // K row this lane feeds to the score MFMA of a 32-key tile (before the tile offset)
  const int krow = 16 * (l32 >> 4) + 8 * ((l32 >> 2) & 1) + 4 * ((l32 >> 3) & 1) + (l32 & 3);
  // transposing V read: this lane's source row and byte offset within a 16-lane group
  const int l16 = lane & 15;
  const int tr_row = l16 >> 2, tr_col = (l16 & 3) * 8;

  // matrix phase of block j: S(j) = K(j) Q^T, then O^T += V(j-1)^T P(j-1)^T
  auto matrix_phase = [&](int j) {
    // Operands are fetched ahead of the MFMAs that consume them (LDS latency is long while the other waves
    // stream their own operands): all K operands first, then the V operands of each 16-key step of P V one step
    // ahead (double-buffered).
    const char *Vs = smem + C::VOFF + ((j - 1) & 1) * C::VBYTES;
    auto vload = [&](int st, i16x8 (&va)[D / 32]) {
      const int t = st >> 1, s2 = st & 1;
      const int k0 = 32 * t + 16 * s2 + 8 * hl + tr_row;  // keys k0 .. k0+3 and k0+4 .. k0+7 of the step
#pragma unroll
      for (int db = 0; db < D / 32; db++) {
        const int pc = (db * 32 + (l32 & 16)) / 8;  // 16-byte piece holding channel D0
        const i16x4 lo = lds_tr16(Vs + voff<D>(k0, pc) + tr_col);
        const i16x4 hi = lds_tr16(Vs + voff<D>(k0 + 4, pc) + tr_col);
        va[db] = i16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
    };
    const bool do_pv = !DUMP && j >= 1;
    i16x8 va[2][D / 32];
    if (j < nblk) {
      const char *Ks = smem + C::KOFF + (j & 1) * C::KBYTES;
      auto kload = [&](int t, int c) {
        const int key = 32 * t + krow;
        return *(const i32x4 *)(Ks + key * C::RB + (((2 * c + hl) ^ kswz<C::RB, C::NP>(key)) * 16));
      };
      if constexpr (C::NCH <= 4) {
        // int8 rows (4 chunks): every K operand at once
        i32x4 ka[2][C::NCH];
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
          for (int c = 0; c < C::NCH; c++) ka[t][c] = kload(t, c);
        if (do_pv) vload(0, va[0]);
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
          for (int c = 0; c < C::NCH; c++) s[t] = mma_qk<QKT>(ka[t][c], qreg[c], c == 0 ? sinit : s[t]);
      } else {
        // 16-bit rows (8 chunks): the operands of chunk c + 2 are read while chunk c multiplies (a 3-deep
        // ring; reading all 16 at once leaves too few registers, and the compiler then waits on each one)
        i32x4 ka[3][2];
#pragma unroll
        for (int c = 0; c < 2; c++)
#pragma unroll
          for (int t = 0; t < 2; t++) ka[c][t] = kload(t, c);
        if (do_pv) vload(0, va[0]);
#pragma unroll
        for (int c = 0; c < C::NCH; c++) {
          if (c + 2 < C::NCH) {
#pragma unroll
            for (int t = 0; t < 2; t++) ka[(c + 2) % 3][t] = kload(t, c + 2);
          }
          // keep the reads here (the scheduler would sink each one to its MFMA and expose its latency)
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int t = 0; t < 2; t++) s[t] = mma_qk<QKT>(ka[c % 3][t], qreg[c], c == 0 ? sinit : s[t]);
        }
      }
    } else if (do_pv) {
      vload(0, va[0]);
    }
    if (do_pv) {
#pragma unroll
      for (int st = 0; st < 4; st++) {
        if (st < 3) vload(st + 1, va[(st + 1) & 1]);
#pragma unroll
        for (int db = 0; db < D / 32; db++) o[db] = mma_pv<VT>(va[st & 1][db], pb[st >> 1][st & 1], o[db]);
      }
    }
  };

  // vector phase of block j: the scores in log2 units (x, masked keys at -inf), the lazy rescale, then
  // P(j) = 2^(x qsc - m) and the row sums
  auto vector_phase = [&](int j) {
    if (j < 0 || j >= nblk) return;
    if constexpr (DUMP) {
      // element i of lane-half hl holds key 64 j + 32 t + 16 (i / 8) + 8 hl + i % 8
      if (qvalid) {
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
          for (int i = 0; i < 16; i++) {
            const int key = j * BK + 32 * t + 16 * (i >> 3) + 8 * hl + (i & 7);
            if (key < p.L) {
              float *dst = (float *)O + ((size_t)h * p.Lq + q) * p.L + key;
              if constexpr (C::QK8) *(int *)dst = s[t][i] - MAGIC;
              else *dst = s[t][i];
            }
          }
      }
      return;
    }
    const int kb = j * BK;
    // x: the scores in log2 units before the query scale. Element i of lane-half hl holds key
    // kb + 32 t + 16 (i / 8) + 8 hl + i % 8.
    auto mask_tile = [&](f32x16 &v, int t) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const int key = kb + 32 * t + 16 * (i >> 3) + 8 * hl + (i & 7);
        bool masked = key >= Lk;
        if constexpr (CAUSAL) masked = masked || key > q + p.causal_off;
        if (masked) v[i] = -INFINITY;
      }
    };
    const bool tail = CAUSAL || kb + BK > Lk;
    f32x16 x[2];
    if constexpr (C::QK8) {
      const float *ksc = (const float *)(smem + C::SOFF) + (j % 3) * BK;
      // all key scales of the block first: one LDS round trip instead of one per group of four keys
      f32x4 k4[2][2][2];
#pragma unroll
      for (int t = 0; t < 2; t++)
#pragma unroll
        for (int s8 = 0; s8 < 2; s8++)
#pragma unroll
          for (int hh = 0; hh < 2; hh++) {
            const int off = 32 * t + 16 * s8 + 8 * hl + 4 * hh;
            k4[t][s8][hh] = *(const f32x4 *)(ksc + off);
          }
#pragma unroll
      for (int t = 0; t < 2; t++) {
        // bit-cast the whole tile (per-element casts of an MFMA result have been miscompiled into a splat)
        x[t] = __builtin_bit_cast(f32x16, s[t]);
#pragma unroll
        for (int s8 = 0; s8 < 2; s8++)
#pragma unroll
          for (int hh = 0; hh < 2; hh++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
              const int i = 8 * s8 + 4 * hh + e;
              x[t][i] = (x[t][i] - MAGICF) * k4[t][s8][hh][e];
            }
      }
      if (tail) {
#pragma unroll
        for (int t = 0; t < 2; t++) mask_tile(x[t], t);
      }
    } else {
      // 16-bit scores are masked in their accumulators (a copy into x before the branch would be made at
      // every block)
      if (tail) {
#pragma unroll
        for (int t = 0; t < 2; t++) mask_tile(s[t], t);
      }
#pragma unroll
      for (int t = 0; t < 2; t++) x[t] = s[t];
    }
    float am[2] = {-INFINITY, -INFINITY};  // two independent chains
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
      for (int i = 0; i < 16; i++) am[t] = fmaxf(am[t], x[t][i]);
    const float amax = fmaxf(am[0], am[1]);
    // lazy running maximum (wave-uniform branch); partner lanes always update together
    if (__any(amax * qsc > m + SLACK)) {
      const float ap = fmaxf(amax, __shfl_xor(amax, 32));
      const float mn = fmaxf(m, ap * qsc);
      const float f = mn == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m - mn);
      m = mn;
      l *= f;
#pragma unroll
      for (int db = 0; db < D / 32; db++)
#pragma unroll
        for (int i = 0; i < 16; i++) o[db][i] *= f;
    }
    const float nm = m == -INFINITY ? 0.0f : -m;
    float ls[2] = {0.0f, 0.0f};  // the row sum of the rounded P that P V uses, two independent chains
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
      for (int i = 0; i < 16; i += 2) {
        const float p0 = __builtin_amdgcn_exp2f(fmaf(x[t][i], qsc, nm));
        const float p1 = __builtin_amdgcn_exp2f(fmaf(x[t][i + 1], qsc, nm));
        const VP2 pr = {(VE)p0, (VE)p1};
        pb[t][i >> 3][i & 7] = pr[0];
        pb[t][i >> 3][(i & 7) + 1] = pr[1];
        ls[t] = sum2<VT>(pr, ls[t]);
      }
    l += ls[0] + ls[1];
  };

  // Ping-pong schedule. Both groups run the same loop body [matrix(j); stage; barrier; vector(j); barrier],
  // group 1 entering it one barrier later, so that in every half-step one group is in its matrix phase and the
  // other in its vector phase (s_barrier counts wave arrivals, not code locations: both groups execute the same
  // number of barriers). Half-step 2j + g is group g's matrix(j); K(j), V(j-1) are read in half-steps 2j, 2j+1.
  // Each group stores its half of K(j+1) and V(j) right after its matrix(j) (half-step 2j + g, after every read
  // of the ring slots they replace) from registers loaded one iteration earlier. Key scales use a 3-deep ring:
  // scale block j is read by group 1 in half-step 2j + 2.
  if (nblk > 0) {
    load_k(0);
    store_k(0);
    load_k(1);
    load_v(0);
  }
  __syncthreads();
  if (grp == 1) __syncthreads();
  for (int j = 0; j <= nblk; j++) {
    // The matrix phase runs at raised wave priority: when both waves of a SIMD are ready to issue, the MFMA
    // stream (the longer dependency chain) goes first and the softmax VALU work fills the gaps.
    __builtin_amdgcn_s_setprio(3);
    matrix_phase(j);
    if (j + 1 < nblk) store_k(j + 1);
    if (j < nblk) store_v(j);
    __builtin_amdgcn_s_setprio(0);
    __syncthreads();
    load_k(j + 2);  // unconditional: blocks past L read as zeros, and the outstanding-load count stays exact
    load_v(j + 1);
    vector_phase(j);
    __syncthreads();
  }
  if (grp == 0) __syncthreads();
  if constexpr (!DUMP) {
    const float lt = l + __shfl_xor(l, 32);
    if (unit >= 0) {
      // partial state of this chunk, unnormalised
      float *wrow = sp.ws + ((size_t)unit * C::BQ + (q - qb * C::BQ)) * (DG + 4);
#pragma unroll
      for (int db = 0; db < DG / 32; db++)
#pragma unroll
        for (int g = 0; g < 4; g++)
          store4<T_F32>((char *)(wrow + db * 32 + 8 * g + 4 * hl), o[db][4 * g], o[db][4 * g + 1], o[db][4 * g + 2],
                        o[db][4 * g + 3]);
      if (hl == 0) {
        wrow[DG] = m;
        wrow[DG + 1] = lt;
      }
      return;
    }
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    if (qvalid) {
      constexpr int OSZ = OT == T_F32 ? 4 : 2;
      const int seq = h / p.seq_heads;
      char *orow = O + (((size_t)seq * p.seq_rows + q) * p.o_stride + (size_t)(h - seq * p.seq_heads) * DG) * OSZ;
#pragma unroll
      for (int db = 0; db < DG / 32; db++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const int d = db * 32 + 8 * g + 4 * hl;
          store4<OT>(orow + d * OSZ, o[db][4 * g] * inv, o[db][4 * g + 1] * inv, o[db][4 * g + 2] * inv,
                     o[db][4 * g + 3] * inv);
        }
    }
  }
}

int esize(int t) { return t == T_I8 ? 1 : t == T_F32 ? 4 : 2; }

}  // namespace

// R partly filled tiles of a last round, cut into s <= CUs / R chunks: R * s <= CUs units of BQ rows of
// (D + 4) floats at D = 128. The allowance per unit is 384 rows (more than any kernel's 256), which also leaves the
// context's scratch room for the h8 GEMM's widened weights of smaller projections.
size_t attention_workspace_max(int cus) { return (size_t)std::max(cus, 1) * 384 * (128 + 4) * sizeof(float); }

namespace {

// Host side: validation (every access the kernel makes must fall inside the
// bound buffers) and launch.
template <int D, int QKT, int VT, int OT, bool CAUSAL, bool DUMP>
int launch_attention(const Pipeline &pl, const Exec &ex, const Arg *args, int nargs, const void *params,
                     uint32_t params_len, std::string *err) {
  using C = Cfg<D == 96 ? 128 : D, QKT>;  // D: the head dim in memory
  if (params_len != sizeof(AttnParams)) {
    *err = "parameter block of " + std::to_string(params_len) + " bytes, expected " +
           std::to_string(sizeof(AttnParams));
    return -1;
  }
  AttnParams p;
  memcpy(&p, params, sizeof p);
  if (p.Lq < 0 || p.L < 1 || p.H < 1 || p.KVH < 1 || p.H % p.KVH || p.q_rows < p.Lq || p.k_rows < p.L ||
      p.o_stride < 0) {
    *err = "bad shape: Lq " + std::to_string(p.Lq) + " L " + std::to_string(p.L) + " H " + std::to_string(p.H) +
           " KVH " + std::to_string(p.KVH) + " q_rows " + std::to_string(p.q_rows) + " k_rows " +
           std::to_string(p.k_rows);
    return -1;
  }
  if (p.seq_heads < 1) p.seq_heads = p.H;
  if (!(p.scale > 0.0f) || !std::isfinite(p.scale)) {
    *err = "softmax scale must be positive and finite";
    return -1;
  }
  const bool qk8 = C::QK8;
  const int need = qk8 ? 7 : 4;
  if (nargs < need) {
    *err = "expected buffers q, k, v, out" + std::string(qk8 ? ", -, q_scale, k_scale" : "");
    return -1;
  }
  for (int i : {0, 1, 2, 3})
    if (!args[i].ptr) {
      *err = "buffer " + std::to_string(i) + " (q, k, v, out) is not bound";
      return -1;
    }
  if (qk8 && (!args[5].ptr || !args[6].ptr)) {
    *err = "int8 scores need q_scale and k_scale";
    return -1;
  }
  auto fits = [&](int i, uint64_t bytes, const char *what) {
    if (bytes > args[i].avail) {
      *err = std::string(what) + " needs " + std::to_string(bytes) + " bytes, its buffer holds " +
             std::to_string(args[i].avail);
      return false;
    }
    return true;
  };
  const uint64_t es = esize(QKT);
  // extents actually read: rows < Lq of every query head, rows < L of every key/value head
  const uint64_t qx = (uint64_t)(p.H - 1) * p.q_rows + p.Lq, kx = (uint64_t)(p.KVH - 1) * p.k_rows + p.L;
  if (!fits(0, qx * D * es, "q") || !fits(1, kx * D * es, "k") || !fits(2, kx * D * 2, "v")) return -1;
  if (qk8 && (!fits(5, qx * 4, "q_scale") || !fits(6, kx * 4, "k_scale"))) return -1;
  // D = 128 without a causal mask: the wave-pipelined kernel (ival[2] = 1)
  constexpr bool CANW = !CAUSAL && D == 128;
  const bool usew = CANW && pl.ival[2] != 0;
  // those kernels address a head's K/V rows (and the blocks their pipelines stage past the end) with 32-bit
  // byte offsets
  if (usew && (uint64_t)(p.L + 4 * BK) * D * 2 > 0xffffffffull) {
    *err = "L = " + std::to_string(p.L) + " keys: too long for 32-bit K/V row offsets";
    return -1;
  }
  if (DUMP) {
    if (nargs < 8 || !args[7].ptr) {
      *err = "the scores hook needs its scores buffer at index 7";
      return -1;
    }
    if (!fits(7, (uint64_t)p.H * p.Lq * p.L * 4, "scores")) return -1;
  }
  if (p.Lq > 0 && (!DUMP || usew)) {
    uint64_t last = 0;
    for (int h = 0; h < p.H; h++) {
      const uint64_t seq = h / p.seq_heads;
      const uint64_t end = ((seq * p.seq_rows + p.Lq - 1) * (uint64_t)p.o_stride + (uint64_t)(h % p.seq_heads) * D + D);
      last = end > last ? end : last;
    }
    if ((uint64_t)p.o_stride < (uint64_t)p.seq_heads * D && p.H > 1 && p.seq_heads > 1) {
      *err = "o_stride " + std::to_string(p.o_stride) + " smaller than seq_heads * D";
      return -1;
    }
    if (!fits(3, last * esize(OT), "out")) return -1;
  }
  // wide accesses: Q, K, V rows are read 16 bytes at a time, O rows written 4 elements at a time
  for (int i : {0, 1, 2})
    if ((uintptr_t)args[i].ptr % 16) {
      *err = std::string(i == 0 ? "q" : i == 1 ? "k" : "v") + " must be 16-byte aligned";
      return -1;
    }
  if ((!DUMP || usew) && ((uintptr_t)args[3].ptr % (4 * esize(OT)) || p.o_stride % 4)) {
    *err = "out must be aligned to 4 elements, and its row stride a multiple of 4 elements";
    return -1;
  }
  if (p.Lq == 0) return 0;
  const int BQ = usew ? WAVE_BQ : C::BQ;
  const int nqb = (p.Lq + BQ - 1) / BQ;
  const long ntiles = (long)nqb * p.H;
  if (ntiles > 0x7fffffffL / 256) {
    *err = "grid too large";
    return -1;
  }
  // Tail split (not for causal masks, whose tiles differ in length, nor for the scores dump): the R tiles of a
  // last, partly filled round of CUs become R * s key chunks, s <= CUs / R, each at least 2 key blocks.
  Split sp{(int)ntiles, 0, 0, nullptr, 0};
  if (usew) sp.rnd = cu_count() / 8;  // these kernels alternate their key order between rounds of an XCD
  const int cus = pl.ival[0] ? cu_count() : 0;
  const int kblocks = (p.L + BK - 1) / BK;
  if (!CAUSAL && (!DUMP || usew) && cus > 0) {
    const int R = (int)(ntiles % cus);
    // chunks per tile: at most CUs / R, at least 2 key blocks each, and as many as the scratch memory holds
    const size_t unit_bytes = (size_t)BQ * (D + 4) * sizeof(float);
    const size_t fit = R ? ex.ws_bytes / (unit_bytes * R) : 0;
    const int smax = R ? (int)std::min<size_t>(std::min(cus / R, kblocks / 2), fit) : 0;
    if (smax >= 2) {
      const int cb = (kblocks + smax - 1) / smax;
      sp.s = (kblocks + cb - 1) / cb;
      sp.cb = cb;
      sp.nfull = (int)ntiles - R;
      sp.ws = (float *)ex.ws;
    }
  }
  const long ngroups = sp.s ? (long)sp.nfull + (ntiles - sp.nfull) * sp.s : ntiles;
  // the scores hook of the older kernels writes the scores instead of the output
  char *out = DUMP && !usew ? args[7].ptr : args[3].ptr;
  if constexpr (CANW) {
    if (usew) return launch_attention_wave(QKT, VT, OT, DUMP, ex, args, p, nqb, sp, err);
  }
  auto kern = attention_kernel<D, QKT, VT, OT, CAUSAL, DUMP>;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS);
    if (e != hipSuccess) {
      *err = std::string("hipFuncSetAttribute: ") + hipGetErrorString(e);
      return -1;
    }
    attr_set = true;
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)ngroups), dim3(C::NT), C::LDS, ex.stream, args[0].ptr, args[1].ptr,
                     args[2].ptr, out, (const float *)args[5].ptr, (const float *)args[6].ptr, p, nqb, sp);
  if (sp.s) {
    const int rows = (int)(ntiles - sp.nfull) * C::BQ;
    hipLaunchKernelGGL((attention_merge<D, OT, C::BQ>), dim3((unsigned)(rows / 4)), dim3(256), 0, ex.stream, sp.ws, args[3].ptr,
                       p, nqb, sp.nfull, sp.s);
  }
  return 0;
}

template <int D, int QKT, int VT, int OT, bool DUMP>
LaunchFn pick_causal(bool causal) {
  if (DUMP) return launch_attention<D, QKT, VT, OT, false, DUMP>;
  return causal ? launch_attention<D, QKT, VT, OT, true, DUMP> : launch_attention<D, QKT, VT, OT, false, DUMP>;
}

template <int D, int QKT, int VT, bool DUMP>
LaunchFn pick_out(int ot, bool causal) {
  switch (ot) {
    case T_BF16: return pick_causal<D, QKT, VT, T_BF16, DUMP>(causal);
    case T_F16: return pick_causal<D, QKT, VT, T_F16, DUMP>(causal);
    default: return pick_causal<D, QKT, VT, T_F32, DUMP>(causal);
  }
}

template <int D, bool DUMP>
LaunchFn pick_types(int qkt, int vt, int ot, bool causal) {
  if (qkt == T_I8) {
    return vt == T_BF16 ? pick_out<D, T_I8, T_BF16, DUMP>(ot, causal) : pick_out<D, T_I8, T_F16, DUMP>(ot, causal);
  }
  return qkt == T_BF16 ? pick_out<D, T_BF16, T_BF16, DUMP>(ot, causal) : pick_out<D, T_F16, T_F16, DUMP>(ot, causal);
}

int type_of(const std::string &s) {
  if (s == "bfloat" || s == "bf16") return T_BF16;
  if (s == "half" || s == "f16") return T_F16;
  if (s == "float" || s == "f32") return T_F32;
  return -1;
}

}  // namespace

// Specialisation macros: HD (head dim: 64, 96 or 128; 96 is the vision tower's
// padded head dim, h3metal/vision.py:34, 129), QK8 (int8 scores), O_T
// (output: half | bfloat | float), CAUSAL, and IN_T (half | bfloat: the type of
// V, and of Q and K without QK8; the reference's inputs are half). The
// reference's tuning macros WM, BK, KPAD, DB, PVORDER, VX, SLACK are accepted
// as integers and do not change the gfx950 kernel (its tiles are its own).
// SPLIT (this build's, default 1): allow the tail split of a partly filled
// last round of workgroups; SPLIT=0 runs every tile whole. GROUPS (this
// build's) 0 or 1: the wave-pipelined kernel for HD 128 without a causal mask
// (the values that selected other kernels for it are refused).
bool make_attention(const std::string &fn, const Macros &m, Pipeline *pl, std::string *err) {
  const bool dump = fn == "attention_scores";
  if (fn != "attention" && !dump) {
    *err = "unknown function (have: attention, attention_scores)";
    return false;
  }
  int hd, qk8, causal, dummy;
  if (!macro_int(m, "HD", 128, &hd, err) || !macro_int(m, "QK8", 0, &qk8, err) ||
      !macro_int(m, "CAUSAL", 0, &causal, err))
    return false;
  for (const char *k : {"WM", "BK", "KPAD", "DB", "PVORDER", "VX", "SLACK", "TG"})
    if (!macro_int(m, k, 0, &dummy, err)) return false;
  int split, groups;
  if (!macro_int(m, "SPLIT", 1, &split, err) || !macro_int(m, "GROUPS", 0, &groups, err)) return false;
  if (groups < 0 || groups > 1) {
    *err = "GROUPS must be 0 or 1 (the wave-pipelined kernel; the paired, ping-pong and two-group kernels that 2-4 "
           "selected for HD 128 without a causal mask are retired)";
    return false;
  }
  for (auto &kv : m) {
    static const char *known[] = {"HD", "QK8", "CAUSAL", "O_T", "IN_T", "WM", "BK", "KPAD", "DB", "PVORDER", "VX",
                                  "SLACK", "TG", "SPLIT", "GROUPS"};
    bool ok = false;
    for (const char *k : known) ok = ok || kv.first == k;
    if (!ok) {
      *err = "unknown macro " + kv.first;
      return false;
    }
  }
  const int ot = type_of(macro_str(m, "O_T", "half"));
  const int it = type_of(macro_str(m, "IN_T", "half"));
  if (ot < 0 || it < 0 || it == T_F32) {
    *err = "O_T must be half|bfloat|float and IN_T half|bfloat";
    return false;
  }
  if (hd != 64 && hd != 96 && hd != 128) {
    *err = "HD " + std::to_string(hd) + " not supported (64, 96 or 128)";
    return false;
  }
  const int qkt = qk8 ? T_I8 : it;
  LaunchFn f;
  if (hd == 128) f = dump ? pick_types<128, true>(qkt, it, ot, causal) : pick_types<128, false>(qkt, it, ot, causal);
  else if (hd == 96) f = dump ? pick_types<96, true>(qkt, it, ot, causal) : pick_types<96, false>(qkt, it, ot, causal);
  else f = dump ? pick_types<64, true>(qkt, it, ot, causal) : pick_types<64, false>(qkt, it, ot, causal);
  pl->launch = f;
  // the kernel the pipeline launches: 1 the wave-pipelined kernel (HD 128 without a causal mask), 0 this file's
  // two-group kernel (every other case)
  const int ksel = hd == 128 && !causal ? 1 : 0;
  pl->threads = ksel == 1 ? WAVE_THREADS : NW * 64;
  pl->ival[0] = split != 0;
  pl->ival[2] = ksel;
  return true;
}

}  // namespace h3
