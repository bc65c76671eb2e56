// Flash attention for gfx950 with two waves per SIMD in ping-pong: the kernel that runs int8-score attention at
// D = 128 without a causal mask (the DiT path's rotated int8 attention). Semantics as the other attention kernels,
// which follow the reference kernel kernels/attention.metal:70-394 (scores in log2 units, key masking at L, int8
// scores scaled by qs_i * ks_j, P rounded to the value type, O divided by the row sum at the end; the row sums add
// the fp32 values of P, as kernels/nax.h:130 row_sum does).
//
// Why this structure. On gfx950 a SIMD runs one wave's MFMAs and another wave's VALU instructions side by side
// without slowing either (measured with s_memtime probes: an MFMA-only wave and a VALU-only wave on one SIMD each
// keep their solo rate), while two waves that both mix MFMAs and VALU work, or one wave that does both, get much
// less overlap, and one wave alone issues VALU work at only ~5-6 cycles per instruction. So the two waves of a SIMD
// take turns: in each half of a key step one of them issues only MFMAs (and the LDS reads that feed them) while the
// other runs only the softmax, and a workgroup barrier swaps them.
//
// Work split. A workgroup is 8 waves (two per SIMD: waves w and w + 4) over 256 query rows of one head: 4 pairs of
// waves, each pair owning 64 query rows (two 32-query MFMA tiles u = 0, 1). Role r = w / 4 of a pair:
//   * scores: S^T = K Q^T for keys 32 r .. 32 r + 31 of each 64-key block and all 64 queries (8 int8 MFMAs), and
//     the softmax of those 2 x 32 x 32 scores;
//   * P V: O^T = V^T P^T for channels 64 r .. 64 r + 63 of the 64 queries over all 64 keys (16 MFMAs), with its own
//     half of P and the partner's half (exchanged through LDS).
// V is read from a transposed copy Vt [KVH][D][Lpad] that the launcher makes first (v_transpose below): an MFMA
// operand of V^T is then 8 consecutive keys of one channel, one 16-byte LDS read, where row-major V needs two
// transposing reads of twice the LDS time each, which eight waves per CU cannot afford.
//
// Step j (block j), two halves separated by workgroup barriers:
//   half 1:  role 0: softmax of block j            role 1: P V of block j - 1, scores of block j + 1
//   half 2:  role 0: P V of block j, scores j + 1   role 1: softmax of block j + 1
// Role 1 runs its softmax one half-step ahead of role 0, so that its half of P(j) is in LDS when role 0 needs it.
// Running maximum: the pair shares one per query row; it is checked lazily after the exponentials (a block is
// accepted when every lane's row sum grew by at most the limit; NaN and inf fail) and a block that fails in any
// wave, and the first and the last block (which holds the key mask), is recomputed by all 8 waves between the
// halves of its step, where both roles have finished its softmax and neither has used its P.
#include "attention_common.h"

#include <algorithm>

// Wave priorities of the two halves (a build variant): 1 raises the softmax half, 2 the MFMA half, 0 neither.
#ifndef PP_PRIO
#define PP_PRIO 0
#endif
#if PP_PRIO == 1
#define PRIO_VALU __builtin_amdgcn_s_setprio(1)
#define PRIO_MFMA __builtin_amdgcn_s_setprio(0)
#elif PP_PRIO == 2
#define PRIO_VALU __builtin_amdgcn_s_setprio(0)
#define PRIO_MFMA __builtin_amdgcn_s_setprio(1)
#else
#define PRIO_VALU
#define PRIO_MFMA
#endif

namespace h3 {
namespace {

// V [KVH][k_rows][128] (rows < L) -> Vt [KVH][128][Lpad], keys L .. Lpad - 1 zero. One workgroup per 64 keys of a
// head: 64 rows of V through LDS (rows padded to 260 bytes: the column reads below are then free of bank conflicts),
// then 128 rows of 64 keys out, 8 lanes per 128-byte row.
// It also writes the seed corrections of the int8 scores, kc = -SEED_F * ks [KVH][Lpad] (0 past L), which the
// attention kernel stages beside the key scales.
__global__ __launch_bounds__(256) void v_transpose(const char *__restrict__ V, char *__restrict__ Vt,
                                                   const float *__restrict__ ks, float *__restrict__ kc, int L,
                                                   int k_rows, int Lpad) {
  constexpr int RS = 260;
  __shared__ __attribute__((aligned(16))) char t[64 * RS];
  const int kb = blockIdx.x, hv = blockIdx.y, tid = threadIdx.x;
  if (tid < 64) {
    const int key = kb * 64 + tid;
    kc[(size_t)hv * Lpad + key] = key < L ? ks[(size_t)hv * k_rows + key] * -0.15915494f : 0.0f;
  }
  const char *src = V + ((size_t)hv * k_rows + (size_t)kb * 64) * 256;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int idx = i * 256 + tid, row = idx >> 4, pc = idx & 15;
    u32x4 v = {0, 0, 0, 0};
    if (kb * 64 + row < L) v = *(const u32x4 *)(src + row * 256 + pc * 16);
    unsigned *d = (unsigned *)(t + row * RS + pc * 16);
    d[0] = v[0];
    d[1] = v[1];
    d[2] = v[2];
    d[3] = v[3];
  }
  __syncthreads();
  char *dst = Vt + ((size_t)hv * 128 * Lpad + (size_t)kb * 64) * 2;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int idx = i * 256 + tid, ch = idx >> 3, pc = idx & 7;
    unsigned short e[8];
#pragma unroll
    for (int k = 0; k < 8; k++) e[k] = *(const unsigned short *)(t + (pc * 8 + k) * RS + ch * 2);
    u32x4 o;
#pragma unroll
    for (int k = 0; k < 4; k++) o[k] = (unsigned)e[2 * k] | ((unsigned)e[2 * k + 1] << 16);
    *(u32x4 *)(dst + (size_t)ch * Lpad * 2 + pc * 16) = o;
  }
}

// P V MFMA with the O accumulator in AGPRs, as assembly (the score MFMAs are builtins with VGPR results that the
// softmax reads). Hazards the compiler cannot see across this assembly: a VALU access of O after these MFMAs is
// preceded by q_fence(o); P (written by VALU) is produced at least one barrier earlier. The build checks the
// generated code for both (h3metal_amd/isa_check.py).
template <int VT>
__device__ __forceinline__ void qpv(f32x16 &acc, i16x8 a, i32x4 b) {
  if constexpr (VT == T_BF16) asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
  else asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
// 18 wait states between the last P V MFMA writing O and a VALU access of O; O is an operand so nothing moves above.
__device__ __forceinline__ void q_fence(f32x16 (&o)[2][2]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 4" : "+a"(o[0][0]), "+a"(o[0][1]), "+a"(o[1][0]), "+a"(o[1][1]));
}
// First int8 score MFMA of a chain onto the seed 1/(2 pi) (an inline constant of srcC); K from VGPRs, Q from AGPRs.
__device__ __forceinline__ i32x16 qmma_seed(i32x4 a, i32x4 b) {
  i32x16 d;
  asm volatile("v_mfma_i32_32x32x32_i8 %0, %1, %2, 0x3e22f983" : "=v"(d) : "v"(a), "a"(b));
  return d;
}

constexpr int NWQ = 8;  // waves per workgroup (two per SIMD)
static_assert(PP_BQ == 256, "4 pairs of 64 query rows");
// int8 score accumulators start from the bits of the float 1/(2 pi): with |q . k| <= 128 * 127^2 < 2^21 the sum
// stays in that float's binade [2^-3, 2^-2), whose ulp is 2^-26, so the accumulator's bits ARE the float
// SEED_F + s * 2^-26, and fma(bits, ks, -SEED_F * ks) = s * ks * 2^-26 replaces an int -> float conversion and a
// multiply (2^26 is folded into the query scale).
constexpr int QSEED_I = 0x3E22F983;
constexpr float QSEED_F = 0.15915494f;
constexpr float QSEED_SCALE = 67108864.0f;  // 2^26

struct CfgQ {
  static constexpr int D = 128;
  static constexpr int RB = 128;  // bytes per K row (int8)
  static constexpr int NP = 8;    // 16-byte pieces per K row (and per Vt row of a block: 64 keys)
  static constexpr int NCH = 4;   // score MFMAs per 32 x 32 tile (32 bytes of D each)
  static constexpr int NRK = 4, NRV = 3;  // ring depths: K and key scales, Vt
  static constexpr int KBYTES = BK * RB, VBYTES = BK * D * 2;
  static constexpr int KOFF = 0;
  static constexpr int VOFF = KOFF + NRK * KBYTES;
  static constexpr int SOFF = VOFF + NRV * VBYTES;
  static constexpr int COFF = SOFF + NRK * BK * 4;  // seed corrections -SEED_F ks, ring like the scales
  static constexpr int POFF = COFF + NRK * BK * 4;
  static constexpr int PBYTES = 4096;  // one wave's P of a block: [query tile][16-key step][lane] x 16 bytes
  static constexpr int FOFF = POFF + 2 * NWQ * PBYTES;  // flags: [slot][wave] bytes
  static constexpr int XOFF = FOFF + 16;                // exchange of block maxima / row sums: [wave][u][32]
  static constexpr int LDS = XOFF + NWQ * 2 * 32 * 4;
  static_assert(LDS <= 160 * 1024, "LDS of one CU");
  static_assert(KBYTES == NWQ * 1024 && VBYTES == 2 * NWQ * 1024, "one K and two Vt loads per wave and block");
};

__device__ __forceinline__ int qufl(int x) { return __builtin_amdgcn_readfirstlane(x); }
// LDS accesses at a byte address (the workgroup's LDS base is passed in by the kernel: a function of its own would
// otherwise load it from memory)
template <class T>
__device__ __forceinline__ T lds_ld(unsigned a) {
  return *(const __attribute__((address_space(3))) T *)(size_t)a;
}
template <class T>
__device__ __forceinline__ void lds_st(unsigned a, T v) {
  *(__attribute__((address_space(3))) T *)(size_t)a = v;
}
__device__ __forceinline__ float quff(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, x)));
}
template <class T>
__device__ __forceinline__ T *qufp(T *x) {
  const unsigned long long v = (unsigned long long)x;
  return (T *)(((unsigned long long)(unsigned)qufl((int)(v >> 32)) << 32) | (unsigned)qufl((int)v));
}

// The body of the kernel for the waves of role R (0: waves 0-3, 1: waves 4-7): a function of its own per role (each
// gets its own register allocation; the two roles run their halves in different orders), called once per wave.
// Its arguments are made wave-uniform again (readfirstlane) for the scalar address arithmetic.
template <int VT, int OT, bool DUMP, int R>
__device__ __attribute__((noinline)) void pp_body(const char *Q_, const char *K_, const char *Vt_, char *O_,
                                                  const float *qs_, const float *ks_, const float *kc_, int *dump_,
                                                  AttnParams p_, int nqb_, Split sp_, int Lpad_, unsigned lds0_) {
  const char *__restrict__ Q = qufp(Q_);
  const char *__restrict__ K = qufp(K_);
  const char *__restrict__ Vt = qufp(Vt_);
  char *__restrict__ O = qufp(O_);
  const float *__restrict__ qs = qufp(qs_);
  const float *__restrict__ ks = qufp(ks_);
  const float *__restrict__ kc = qufp(kc_);
  int *__restrict__ dump = qufp(dump_);
  const AttnParams p{qufl(p_.Lq), qufl(p_.L), qufl(p_.H), qufl(p_.KVH), qufl(p_.q_rows), qufl(p_.k_rows),
                     qufl(p_.o_stride), quff(p_.scale), qufl(p_.causal_off), qufl(p_.seq_heads), qufl(p_.seq_rows)};
  const int nqb = qufl(nqb_), Lpad = qufl(Lpad_);
  const Split sp{qufl(sp_.nfull), qufl(sp_.s), qufl(sp_.cb), qufp(sp_.ws), qufl(sp_.rnd)};
  using C = CfgQ;
  constexpr int D = C::D;
  using VE = typename Vec8<VT>::elem;
  using VP2 = typename Vec8<VT>::pair;
  const unsigned lds0 = (unsigned)qufl((int)lds0_);

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
  const int q0 = qb * PP_BQ + pr * 64 + l32;  // this lane's query rows: q0 + 32 u

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
    qsw[u] = qsc[u] * QSEED_SCALE;
  }

  int key0 = 0, Lk = p.L;
  if (unit >= 0) {
    key0 = (unit % sp.s) * sp.cb * BK;
    Lk = min(p.L, key0 + sp.cb * BK) - key0;
  }
  const char *Kh = K + ((size_t)kvh * p.k_rows + key0) * C::RB;
  const char *Vth = Vt + ((size_t)kvh * D * Lpad + key0) * 2;
  const float *ksh = ks + (size_t)kvh * p.k_rows + key0;
  const float *kch = kc + (size_t)kvh * Lpad + key0;
  const int nblk = Lk > 0 ? (Lk + BK - 1) / BK : 0;
  auto kblk = [&](int j) { return __builtin_amdgcn_readfirstlane(rev && j < nblk - 1 ? nblk - 2 - j : j); };

  // -- LDS-direct staging: each wave loads 1 KB of K, 2 KB of Vt and (every wave, to the same place) the 64 key
  // scales of a block. The K and scale descriptors cover this workgroup's Lk rows (rows past it, and blocks past
  // the end, read as zero); the Vt descriptor covers the rest of this head's Vt, whose keys past L are zero.
  auto rsrc = [&](const void *base, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, __builtin_amdgcn_readfirstlane((int)bytes),
                                             0x00020000);
  };
  const __amdgpu_buffer_rsrc_t rk = rsrc(Kh, (unsigned)max(0, Lk) * C::RB);
  const __amdgpu_buffer_rsrc_t rv = rsrc(Vth, (unsigned)(D * Lpad - key0) * 2u);
  const __amdgpu_buffer_rsrc_t rs = rsrc(ksh, (unsigned)max(0, Lk) * 4u);
  const __amdgpu_buffer_rsrc_t rc = rsrc(kch, (unsigned)(Lpad - key0) * 4u);
  unsigned kgo, vgo[2];
  {
    const int o = w * 1024 + 16 * lane;
    const int row = o / C::RB, slot = (o / 16) % C::NP;
    kgo = row * C::RB + (slot ^ kswz<C::RB, C::NP>(row)) * 16;
#pragma unroll
    for (int rr = 0; rr < 2; rr++) {
      // Vt block in LDS: [channel][64 keys], 128-byte rows, 16-byte piece p of row ch at slot p ^ ((ch / 2) % 8)
      const int ov = (rr * NWQ + w) * 1024 + 16 * lane;
      const int ch = ov >> 7, sl = (ov >> 4) & 7;
      vgo[rr] = (unsigned)ch * (unsigned)Lpad * 2u + (unsigned)((sl ^ ((ch >> 1) & 7)) * 16);
    }
  }
  // staging load i for K block kb (i = 0: this wave's K piece, 1: the scales, 4: the corrections) or Vt block vb
  // (i = 2, 3: this wave's pieces)
  auto stage = [&](int i, int kb, int vb) {
    if (i == 0) {
      dma16(lds0 + C::KOFF + (kb % C::NRK) * C::KBYTES + w * 1024, kgo + (unsigned)kblk(kb) * C::KBYTES, rk);
    } else if (i == 1) {
      dma4(lds0 + C::SOFF + (kb % C::NRK) * BK * 4, lane * 4 + (unsigned)kblk(kb) * (BK * 4), rs);
    } else if (i == 4) {
      dma4(lds0 + C::COFF + (kb % C::NRK) * BK * 4, lane * 4 + (unsigned)kblk(kb) * (BK * 4), rc);
    } else {
      const int rr = i - 2;
      dma16(lds0 + C::VOFF + (vb % C::NRV) * C::VBYTES + (rr * NWQ + w) * 1024, vgo[rr] + (unsigned)kblk(vb) * 128u,
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
  float m[2], nmv[2];
#pragma unroll
  for (int u = 0; u < 2; u++) {
    m[u] = -INFINITY;
    nmv[u] = 0.0f;
  }
  // Row sums of this wave's half of P, accumulated on the matrix pipe: a 16x16x32 MFMA takes a packed P register
  // of query tile u (as its B operand: column n = lane % 16, key group lane / 16) against the selector `sel` (row 0
  // ones on key groups 0 and 2, which hold query n; row 1 on groups 1 and 3, query n + 16), so that in lanes 0-15
  // element 0 of lsum[u] is the running sum of query n and element 1 that of query n + 16 (rows 2-15 stay 0).
  f32x4 lsum[2];
#pragma unroll
  for (int u = 0; u < 2; u++) lsum[u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  i32x4 sel;
  {
    const int m16 = lane & 15, g = lane >> 4;
    const int one = (m16 == 0 && (g & 1) == 0) || (m16 == 1 && (g & 1) == 1) ? (VT == T_F16 ? 0x3C003C00 : 0x3F803F80) : 0;
    sel = i32x4{one, one, one, one};
  }
  auto rowsum = [&](int u, i32x4 pp) {
    if constexpr (VT == T_BF16)
      lsum[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, sel), __builtin_bit_cast(bf16x8, pp),
                                                       lsum[u], 0, 0, 0);
    else
      lsum[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, sel), __builtin_bit_cast(f16x8, pp),
                                                      lsum[u], 0, 0, 0);
  };
  i32x16 s[2];     // [u] scores of this wave's key half
  i32x4 pb[2][2];  // [u][16-key step within the half] own P, packed 16-bit
#pragma unroll
  for (int u = 0; u < 2; u++) {
#pragma unroll
    for (int i = 0; i < 16; i++) s[u][i] = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) pb[u][i >> 2][i & 3] = 0;
  }

  // LDS addressing of the MFMA operands
  const int krow = 16 * (l32 >> 4) + 8 * ((l32 >> 2) & 1) + 4 * ((l32 >> 3) & 1) + (l32 & 3);
  unsigned kbase[C::NCH], vtb[2], vpo[4];
#pragma unroll
  for (int c = 0; c < C::NCH; c++)
    kbase[c] = 32 * r * C::RB + krow * C::RB + (((2 * c + hl) ^ kswz<C::RB, C::NP>(krow)) * 16);
#pragma unroll
  for (int c = 0; c < 2; c++) vtb[c] = (unsigned)((32 * (2 * r + c) + l32) * 128);
#pragma unroll
  for (int st = 0; st < 4; st++) vpo[st] = (unsigned)(((2 * st + hl) ^ ((l32 >> 1) & 7)) * 16);
  // Vt(j) operand (A of O^T = V^T P^T): channel tile 2 r + c, keys 16 st + 8 hl .. + 7 of the block (one read)
  auto vread = [&](int j, int st, int c) {
    return lds_ld<i16x8>(lds0 + C::VOFF + ((j + C::NRV) % C::NRV) * C::VBYTES + vtb[c] + vpo[st]);
  };
  auto kread = [&](int j, int c) {  // K(j), chunk c of this wave's key half
    return lds_ld<i32x4>(lds0 + C::KOFF + (j % C::NRK) * C::KBYTES + kbase[c]);
  };
  auto sread = [&](int j, int g) {  // scales of K(j): keys 32 r + 16 (g / 2) + 8 hl + 4 (g % 2) + e
    return lds_ld<f32x4>(lds0 + C::SOFF + 4 * ((j % C::NRK) * BK + 32 * r + 16 * (g >> 1) + 8 * hl + 4 * (g & 1)));
  };
  auto cread = [&](int j, int g) {  // their seed corrections
    return lds_ld<f32x4>(lds0 + C::COFF + 4 * ((j % C::NRK) * BK + 32 * r + 16 * (g >> 1) + 8 * hl + 4 * (g & 1)));
  };
  auto paddr = [&](int j, int wv, int u, int s2) {
    return C::POFF + ((((j + 2) & 1) * NWQ + wv) * 4 + u * 2 + s2) * 1024 + lane * 16;
  };
  auto pwrite = [&](int j) {
#pragma unroll
    for (int u = 0; u < 2; u++)
#pragma unroll
      for (int s2 = 0; s2 < 2; s2++) lds_st<i32x4>(lds0 + paddr(j, w, u, s2), pb[u][s2]);
  };
  auto pread = [&](int j, int wv, int u, int s2) { return lds_ld<i32x4>(lds0 + paddr(j, wv, u, s2)); };
  auto dump_scores = [&](const i32x16 &acc, int j, int u) {
    if constexpr (DUMP) {
      const int q = q0 + 32 * u;
      if (q < p.Lq && j < nblk) {
        const i32x16 a = acc - QSEED_I;
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

  f32x4 k4[4], c4[4];  // key scales of the block whose softmax runs next, and their seed corrections -SEED_F ks

  // Scores of block jn (this wave's key half, both query tiles) onto the seed, from K operands in ka.
  auto score_mfmas = [&](const i32x4 (&ka)[C::NCH]) {
#pragma unroll
    for (int c = 0; c < C::NCH; c++)
#pragma unroll
      for (int u = 0; u < 2; u++) {
        if (c == 0) s[u] = qmma_seed(ka[0], qreg[u][0]);
        else s[u] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ka[c], qreg[u][c], s[u], 0, 0, 0);
      }
  };
  auto scale_prep = [&](int jn) {  // key scales of block jn and their seed corrections
#pragma unroll
    for (int g = 0; g < 4; g++) {
      k4[g] = sread(jn, g);
      c4[g] = cread(jn, g);
    }
  };
  auto scores = [&](int jn) {
    i32x4 ka[C::NCH];
#pragma unroll
    for (int c = 0; c < C::NCH; c++) ka[c] = kread(jn, c);
    score_mfmas(ka);
  };

  // Operands of one 16-key step st of a P V of block jb: Vt of both channel tiles, and P of both query tiles where
  // it comes from LDS (the partner's half, and role 1's own half, which its next softmax overwrites in registers
  // first). Key step st belongs to role st / 2.
  struct StepOps {
    i16x8 v[2];
    i32x4 p[2];
  };
  auto step_ops = [&](int jb, int st, StepOps &op) {
    op.v[0] = vread(jb, st, 0);
    op.v[1] = vread(jb, st, 1);
    if (!(R == 0 && st < 2)) {
      const int wv = st / 2 == R ? w : wp;
#pragma unroll
      for (int u = 0; u < 2; u++) op.p[u] = pread(jb, wv, u, st & 1);
    }
  };
#define SB __builtin_amdgcn_sched_barrier(0)
  // The MFMA half: P V of block jb (first key step's operands in `pre`), then the scores and key scales of block
  // js (if has_s). Each step's LDS operands are read one step ahead, the K operands during the second and third
  // steps; the MFMAs of a step are issued together.
  auto mphase = [&](int jb, int js, bool has_s) {
    StepOps cur, nxt;
    step_ops(jb, 0, cur);
    i32x4 ka[C::NCH];
#pragma unroll
    for (int st = 0; st < 4; st++) {
      if (st < 3) step_ops(jb, st + 1, nxt);
      if (has_s && st == 1) {
        ka[0] = kread(js, 0);
        ka[1] = kread(js, 1);
      }
      if (has_s && st == 2) {
        ka[2] = kread(js, 2);
        ka[3] = kread(js, 3);
      }
      SB;
#pragma unroll
      for (int u = 0; u < 2; u++) {
        const i32x4 pp = R == 0 && st < 2 ? pb[u][st] : cur.p[u];
        qpv<VT>(o[u][0], cur.v[0], pp);
        qpv<VT>(o[u][1], cur.v[1], pp);
        if (st / 2 == R) rowsum(u, pp);  // this wave's half of P
      }
      SB;
      cur = nxt;
    }
    if (has_s) {
      score_mfmas(ka);
      scale_prep(js);
    }
    SB;
  };

  auto p_ok = [&](const i32x4 (&pp)[2][2]) {
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    u16x2 mx = __builtin_bit_cast(u16x2, pp[0][0][0]);
#pragma unroll
    for (int k = 1; k < 16; k++) mx = __builtin_elementwise_max(mx, __builtin_bit_cast(u16x2, pp[k >> 3][(k >> 2) & 1][k & 3]));
    constexpr unsigned short LIM = VT == T_F16 ? 0x7800 : 0x4E80;  // 2^15 as f16, 2^30 as bf16
    return mx[0] < LIM && mx[1] < LIM;
  };

  // The softmax of block j (its scores in s): P into pb and LDS, and this wave's flag for the lazy-maximum check
  // of block j (some P of the block at or above the limit, 2^30 with bf16 P and 2^15 with f16 P, whose largest
  // finite value is 65504; or inf or NaN).
  auto softmax = [&](int j) {
    dump_scores(s[0], j, 0);
    dump_scores(s[1], j, 1);
    f32x16 x[2] = {__builtin_bit_cast(f32x16, s[0]), __builtin_bit_cast(f32x16, s[1])};
    // stage by stage over all 32 values of the lane, so that no instruction waits for the one just before it (a
    // lone wave issues a dependent VALU instruction at about half the rate of an independent one)
#pragma unroll
    for (int u = 0; u < 2; u++)
#pragma unroll
      for (int i = 0; i < 16; i++) x[u][i] = fmaf(x[u][i], k4[i >> 2][i & 3], c4[i >> 2][i & 3]);
    SB;
#pragma unroll
    for (int u = 0; u < 2; u++)
#pragma unroll
      for (int i = 0; i < 16; i++) x[u][i] = fmaf(x[u][i], qsw[u], nmv[u]);
    SB;
#pragma unroll
    for (int u = 0; u < 2; u++)
#pragma unroll
      for (int i = 0; i < 16; i++) x[u][i] = __builtin_amdgcn_exp2f(x[u][i]);
    SB;
#pragma unroll
    for (int u = 0; u < 2; u++)
#pragma unroll
      for (int i = 0; i < 16; i += 2) {
        const VP2 v2 = {(VE)x[u][i], (VE)x[u][i + 1]};
        pb[u][i >> 3][(i & 7) >> 1] = __builtin_bit_cast(int, v2);
      }
    pwrite(j);
    // the lazy-maximum check on the packed P: its largest 16-bit pattern (for P >= 0 the unsigned order of the
    // bits is the order of the values, with inf and NaN above every finite value) against the limit's
    const bool wbad = __builtin_amdgcn_ballot_w64(!p_ok(pb)) != 0;
    if (lane == 0) lds_st<unsigned char>(lds0 + C::FOFF + (j & 1) * 8 + w, wbad ? 1 : 0);
  };

  // rare (uniform over the workgroup, between the halves of step j): block j again with the pair's exact maximum
  auto recompute = [&](int j) {
    q_fence(o);  // P V MFMAs may still be writing O
    const bool mask = j == nblk - 1;
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
      if (hl == 0) lds_st<float>(lds0 + C::XOFF + 4 * ((w * 2 + u) * 32 + l32), bm[u]);
      __builtin_amdgcn_sched_barrier(0);
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 2; u++) {
      const float pm = fmaxf(bm[u], lds_ld<float>(lds0 + C::XOFF + 4 * ((wp * 2 + u) * 32 + l32))) * qsc[u];
      const float mn = fmaxf(m[u], pm);
      const float f = (m[u] == -INFINITY || mn == -INFINITY) ? 1.0f : __builtin_amdgcn_exp2f(m[u] - mn);
      m[u] = mn;
      // the row sums of queries n and n + 16 (lanes 0-15) take the factors of those queries' lanes
      lsum[u][0] *= f;
      lsum[u][1] *= __shfl(f, (lane & 15) + 16);
      // one 16-register tile at a time (the tiles live in AGPRs: a VALU multiply goes through VGPRs)
#pragma unroll
      for (int c = 0; c < 2; c++) {
#pragma unroll
        for (int i = 0; i < 16; i++) o[u][c][i] *= f;
        asm volatile("" : "+a"(o[u][c]));
      }
      const float nm = mn == -INFINITY ? 0.0f : -mn;
      nmv[u] = nm;
      rescore(u, [&](const f32x16 &x) {
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
          const float p0 = __builtin_amdgcn_exp2f(fmaf(x[i], qsc[u], nm));
          const float p1 = __builtin_amdgcn_exp2f(fmaf(x[i + 1], qsc[u], nm));
          const VP2 pp = {(VE)p0, (VE)p1};
          pb[u][i >> 3][(i & 7) >> 1] = __builtin_bit_cast(int, pp);
        }
      });
      __builtin_amdgcn_sched_barrier(0);
    }
    pwrite(j);
    asm volatile("s_nop 2" ::: "memory");  // VALU writes of O before the next MFMA reads it
    __syncthreads();                       // the partner reads the recomputed P
  };

#ifdef PP_TIMING
  // timing-only builds: shader-clock ticks of [half 1, wait at the middle barrier, half 2, wait at the end barrier,
  // rare branches], written to the output's first bytes at the end (workgroup b, wave w at 8 (8 b + w))
  unsigned long long tph[6] = {0, 0, 0, 0, 0, 0}, tlast = 0;
  auto tick = [&](int k) {
    __builtin_amdgcn_sched_barrier(0);
    const unsigned long long now = __builtin_amdgcn_s_memtime();
    __builtin_amdgcn_sched_barrier(0);
    if (k >= 0) tph[k] += now - tlast;
    tlast = now;
  };
#else
  auto tick = [](int) {};
#endif
  // Staging. Role 0 at the end of its MFMA half of step j: its pieces of K(j + 3) (slot of K(j - 1), last read in
  // the recompute of step j - 1), the scales and corrections of block j + 3 and its pieces of Vt(j + 2) (slot of Vt(j - 1), whose
  // last reader, role 1, read it in half 1 of step j); waited for before the end barrier of step j + 1. Role 1 at
  // the end of its MFMA half of step j: its pieces of K(j + 3) and of Vt(j + 1) (slot of Vt(j - 2)); waited for
  // before the middle barrier of step j + 1.
  auto stage0 = [&](int j) {
    stage(0, j + 3, j + 2); stage(1, j + 3, j + 2); stage(4, j + 3, j + 2); stage(2, j + 3, j + 2); stage(3, j + 3, j + 2);
  };
  auto stage1 = [&](int j) { stage(0, j + 3, j + 1); stage(2, j + 3, j + 1); stage(3, j + 3, j + 1); };
  if (nblk > 0) {
    // prologue: K, scales of blocks 0, 1 and Vt of block 0; the scores of block 0; the first staging loads (role 0:
    // K, scales 2 and Vt 1; role 1: K 2), and role 1's softmax of block 0. Role 1's P V of block -1 (in step 0)
    // reads Vt ring slot 2 and P slot 1, zeroed here, so that every step runs one code path; so do the scores of
    // the block past the last (zero K rows), whose softmax is never used.
#pragma unroll
    for (int i = 0; i < 2; i++)
      lds_st<i32x4>(lds0 + C::VOFF + 2 * C::VBYTES + (i * NWQ + w) * 1024 + lane * 16, i32x4{0, 0, 0, 0});
#pragma unroll
    for (int i = 0; i < 4; i++) lds_st<i32x4>(lds0 + C::POFF + ((NWQ + w) * 4 + i) * 1024 + lane * 16, i32x4{0, 0, 0, 0});
    stage(0, 0, 0); stage(1, 0, 0); stage(4, 0, 0);
    stage(0, 1, 0); stage(1, 1, 0); stage(4, 1, 0);
    stage(2, 0, 0); stage(3, 0, 0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    scores(0);
    scale_prep(0);
    SB;
    if constexpr (R == 0) {
      stage0(-1);
    } else {
      stage(0, 2, 0);
      softmax(0);
    }
    __syncthreads();
    for (int j = 0; j < nblk; j++) {
      tick(-1);
      // ---- half 1
      if constexpr (R == 0) {
        PRIO_VALU;
        softmax(j);
        PRIO_MFMA;
      } else {
        mphase(j - 1, j + 1, true);
        tick(5);
        stage1(j);
        asm volatile("s_waitcnt vmcnt(3)" ::: "memory");  // this wave's staging of step j - 1 has landed
      }
      SB;
      tick(0);
      __syncthreads();
      tick(1);
      {
        const unsigned long long flags = lds_ld<unsigned long long>(lds0 + C::FOFF + (j & 1) * 8);
        if (__builtin_expect(j == 0 || j == nblk - 1 ||
                                 __builtin_amdgcn_readfirstlane((unsigned)(flags | (flags >> 32))) != 0,
                             0)) {
          recompute(j);
          tick(4);
          if constexpr (R == 1) {
            // the scores and key scales of block j + 1 again (out of the branch's live registers)
            scores(j + 1);
            scale_prep(j + 1);
          }
        }
      }
      SB;
      // ---- half 2
      if constexpr (R == 0) {
        mphase(j, j + 1, true);
        tick(5);
        stage0(j);
        // this wave's loads of the previous step have landed (this step's 5 may still be in flight)
        asm volatile("s_waitcnt vmcnt(5)" ::: "memory");
      } else {
        PRIO_VALU;
        softmax(j + 1);
        PRIO_MFMA;
      }
      SB;
      tick(2);
      __syncthreads();
      tick(3);
    }
    if constexpr (R == 1) {
      // P V of the last block
      mphase(nblk - 1, 0, false);
      q_fence(o);  // before any copy of O the compiler might place after these MFMAs
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // loads past the last block land before the exit
    q_fence(o);
  }

#ifdef PP_TIMING
  if (lane == 0) {
    long long *tp = (long long *)O + ((size_t)blockIdx.x * NWQ + w) * 8;
    for (int k = 0; k < 6; k++) tp[k] = (long long)tph[k];
    tp[7] = nblk;
  }
  return;
#endif
  // row sums: this wave's half (two lanes per query), then the partner's through LDS
  float lt[2];
#pragma unroll
  for (int u = 0; u < 2; u++) {
    // query l32 of tile u: element 0 of lane l32 (l32 < 16) or element 1 of lane l32 - 16
    const float a = __shfl(lsum[u][0], l32 & 15), b2 = __shfl(lsum[u][1], l32 & 15);
    lt[u] = l32 < 16 ? a : b2;
    if (hl == 0) lds_st<float>(lds0 + C::XOFF + 4 * ((w * 2 + u) * 32 + l32), lt[u]);
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < 2; u++) lt[u] += lds_ld<float>(lds0 + C::XOFF + 4 * ((wp * 2 + u) * 32 + l32));

#pragma unroll
  for (int u = 0; u < 2; u++) {
    const int q = q0 + 32 * u;
    if (unit >= 0) {
      float *wrow = sp.ws + ((size_t)unit * PP_BQ + (q - qb * PP_BQ)) * (D + 4);
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

#undef SB

template <int VT, int OT, bool DUMP>
__global__ __launch_bounds__(NWQ * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attention_pp_kernel(const char *__restrict__ Q, const char *__restrict__ K, const char *__restrict__ Vt,
                         char *__restrict__ O, const float *__restrict__ qs, const float *__restrict__ ks,
                         const float *__restrict__ kc, int *__restrict__ dump, AttnParams p, int nqb, Split sp,
                         int Lpad) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const unsigned lds0 = (unsigned)(size_t)(__attribute__((address_space(3))) char *)smem;
  if (__builtin_amdgcn_readfirstlane(threadIdx.x >> 6) < 4)
    pp_body<VT, OT, DUMP, 0>(Q, K, Vt, O, qs, ks, kc, dump, p, nqb, sp, Lpad, lds0);
  else
    pp_body<VT, OT, DUMP, 1>(Q, K, Vt, O, qs, ks, kc, dump, p, nqb, sp, Lpad, lds0);
}

}  // namespace

// scratch of a launch: Vt [KVH][128][Lpad] (16-bit), then the corrections [KVH][Lpad] (fp32)
static size_t vt_part(const AttnParams &p, size_t lpad) { return ((size_t)p.KVH * 128 * lpad * 2 + 255) / 256 * 256; }
size_t attention_pp_vt_bytes(const AttnParams &p) {
  const size_t lpad = ((size_t)p.L + BK - 1) / BK * BK;
  return vt_part(p, lpad) + ((size_t)p.KVH * lpad * 4 + 255) / 256 * 256;
}

int launch_attention_pp(int vt, int ot, bool dump, const Exec &ex, const Arg *args, const AttnParams &p, int nqb,
                        const Split &sp, char *vtbuf, std::string *err) {
  const int lpad = (p.L + BK - 1) / BK * BK;
  float *kcbuf = (float *)(vtbuf + vt_part(p, (size_t)lpad));
  hipLaunchKernelGGL(v_transpose, dim3((unsigned)(lpad / BK), (unsigned)p.KVH), dim3(256), 0, ex.stream, args[2].ptr,
                     vtbuf, (const float *)args[6].ptr, kcbuf, p.L, p.k_rows, lpad);
  auto run = [&](auto kern) -> int {
    static bool attr_set[4][4][2] = {};
    bool &set = attr_set[vt][ot][dump];
    if (!set) {
      hipError_t e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, CfgQ::LDS);
      if (e != hipSuccess) {
        *err = std::string("hipFuncSetAttribute: ") + hipGetErrorString(e);
        return -1;
      }
      set = true;
    }
    const long ntiles = (long)nqb * p.H;
    const long ngroups = sp.s ? (long)sp.nfull + (ntiles - sp.nfull) * sp.s : ntiles;
    hipLaunchKernelGGL(kern, dim3((unsigned)ngroups), dim3(NWQ * 64), CfgQ::LDS, ex.stream, args[0].ptr, args[1].ptr,
                       vtbuf, args[3].ptr, (const float *)args[5].ptr, (const float *)args[6].ptr, kcbuf,
                       dump ? (int *)args[7].ptr : nullptr, p, nqb, sp, lpad);
    if (sp.s) {
      const int rows = (int)(ntiles - sp.nfull) * PP_BQ;
      switch (ot) {
        case T_BF16:
          hipLaunchKernelGGL((attention_merge<128, T_BF16, PP_BQ>), dim3((unsigned)(rows / 4)), dim3(256), 0,
                             ex.stream, sp.ws, args[3].ptr, p, nqb, sp.nfull, sp.s);
          break;
        case T_F16:
          hipLaunchKernelGGL((attention_merge<128, T_F16, PP_BQ>), dim3((unsigned)(rows / 4)), dim3(256), 0,
                             ex.stream, sp.ws, args[3].ptr, p, nqb, sp.nfull, sp.s);
          break;
        default:
          hipLaunchKernelGGL((attention_merge<128, T_F32, PP_BQ>), dim3((unsigned)(rows / 4)), dim3(256), 0,
                             ex.stream, sp.ws, args[3].ptr, p, nqb, sp.nfull, sp.s);
      }
    }
    return 0;
  };
  auto with_ot = [&](auto v_c, auto d_c) -> int {
    constexpr int VT = decltype(v_c)::value;
    constexpr bool DUMP = decltype(d_c)::value;
    switch (ot) {
      case T_BF16: return run(attention_pp_kernel<VT, T_BF16, DUMP>);
      case T_F16: return run(attention_pp_kernel<VT, T_F16, DUMP>);
      default: return run(attention_pp_kernel<VT, T_F32, DUMP>);
    }
  };
  using B16 = std::integral_constant<int, T_BF16>;
  using F16 = std::integral_constant<int, T_F16>;
  if (vt == T_BF16) return dump ? with_ot(B16{}, std::true_type{}) : with_ot(B16{}, std::false_type{});
  return dump ? with_ot(F16{}, std::true_type{}) : with_ot(F16{}, std::false_type{});
}

}  // namespace h3
