// int8 matrix product of the projections around attention, for gfx950:
//   v[m][n] = sa[m] * sw[n] * sum_k A[m][k] * W[n][k]      (A, W int8, row-major in k; int32 accumulation)
// with the epilogues of the reference kernel gemm (kernels/gemm.metal, weight format Q8 = WFMT 1, :1-40,
// :118-261; parameters kernels/params.h:7-16; launcher h3metal/ops.py:124-174):
//   EPI 0: C[m][n] = OUT_T(v + bias[n])
//   EPI 1: X[m][n] += gate[rtype[m]][n] * (v + bias[n])    (X float, the residual stream)
// Every float step is one IEEE-rounded operation in the reference's order, float(acc) * sa[m] * sw[n], then
// + bias, then (EPI 1) gate * v and + X (this file is compiled without FMA contraction), so a float32
// restatement reproduces the outputs bit for bit; the int32 accumulators are exact.
//
// gfx950 design: a workgroup of 8 waves computes a 256 x 256 tile of C on v_mfma_i32_32x32x32_i8; wave
// (wm, wn) owns rows 64 wm .. +63 and columns 128 wn .. +127 (2 x 4 MFMA tiles, 128 accumulator registers).
// K advances in steps of 64 bytes through 4 LDS stages of 32 KB (A rows, then W rows), filled by LDS-direct
// 16-byte buffer loads four steps ahead (rows past M or N read as zero); one barrier per step, and the operands
// of the next step are read from LDS while the MFMAs of the current one run. LDS rows are 64 bytes; 16-byte
// piece p of row r sits at slot p ^ ((r / 4) % 4), which makes the operand reads (16 rows at one piece per
// 16-lane pass) bank-conflict free. Workgroups are ordered so that each XCD (own L2) sweeps bands of 4 row
// tiles across the column tiles.
// Epilogues: for the plain outputs the MFMAs compute C^T (W rows as the A operand), so an accumulator lane
// holds one row of C and 4 consecutive columns per group of 4 elements; the tile goes through LDS (float
// outputs half a tile at a time) and leaves as 16-byte row stores. The residual form keeps C in the
// accumulators (a lane holds one column) and reads X, writes X per wave without barriers, 128 contiguous bytes
// of two rows per access, so one wave's epilogue overlaps the other waves' MFMAs.
#include "h3hip_internal.h"

#include <algorithm>
#include <cstring>
#include <type_traits>

namespace h3 {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// operand types of a kernel: int8 (q8), half (f16, and h8 after its weights are widened), bfloat (bf16)
enum { A_I8 = 0, A_F16 = 1, A_BF16 = 2 };
// epilogue scaling: sa[m] * sw[n] (q8), sw[n] (h8), none (f16, bf16)
enum { S_ROW_COL = 0, S_COL = 1, S_NONE = 2 };

enum { T_BF16 = 1, T_F16 = 2, T_F32 = 3 };

template <int AT>
using AccOf = typename std::conditional<AT == A_I8, i32x16, f32x16>::type;

// one 32 x 32 product over a 32-byte K slice per lane half (32 int8 or 16 16-bit values of K)
template <int AT>
__device__ __forceinline__ AccOf<AT> mma(i32x4 a, i32x4 b, AccOf<AT> c) {
  if constexpr (AT == A_I8) return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
  else if constexpr (AT == A_F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

constexpr int KS = 64;                           // K bytes per step
constexpr int NWG = 8;                           // waves per workgroup
constexpr int WGN = 2, WGM = NWG / WGN;          // waves along the columns and the rows of the tile
constexpr int SW = 4;                            // row tiles per band of the tile order
constexpr int NST = 4;                           // LDS stages
// Tile configurations: 256 x 256 (the main grid) and 128 x 128 (the rows of a last, mostly empty round of
// tiles, run as a second launch of their own)
template <int TM_, int TN_>
struct GTile {
  static constexpr int TM = TM_, TN = TN_;                       // tile rows, columns
  static constexpr int WTM = TM / WGM, WTN = TN / WGN;           // wave tile
  static constexpr int MI = WTM / 32, NJ = WTN / 32;             // 32 x 32 MFMA tiles per wave
  static constexpr int NQA = TM / NWG / 16, NQW = TN / NWG / 16;  // 16-row LDS-direct loads per wave and step
  static constexpr int LPS = NQA + NQW;                          // loads per wave and step
  static constexpr int STAGE = (TM + TN) * KS;                   // LDS bytes per stage
  template <int OT>
  static constexpr int lds_bytes() {
    return std::max(NST * STAGE, OT == T_F32 ? TM / 2 * (TN * 4 + 16) : TM * (TN * 2 + 16));
  }
};
using TileBig = GTile<256, 256>;
using TileSmall = GTile<128, 128>;

// 16-byte piece p of LDS row r (64 bytes) sits at slot p ^ ((r / 4) % 4)
__device__ __forceinline__ int swz(int row, int piece) { return row * KS + ((piece ^ ((row >> 2) & 3)) << 4); }


template <int OT>
__device__ __forceinline__ void store_out(char *p, float v) {
  if constexpr (OT == T_F32) *(float *)p = v;
  else if constexpr (OT == T_BF16) *(__bf16 *)p = (__bf16)v;
  else *(_Float16 *)p = (_Float16)v;
}

template <int OT, int EPI, bool HAS_BIAS, int AT, int SM, class TL>
__global__ __launch_bounds__(NWG * 64) __attribute__((amdgpu_waves_per_eu(2))) void gemm_kernel(const char *__restrict__ A,
                                                           const char *__restrict__ W,
                                                           const float *__restrict__ sw, const float *__restrict__ sa,
                                                           char *__restrict__ out, const float *__restrict__ bias,
                                                           const unsigned char *__restrict__ rtype,
                                                           const float *__restrict__ gate, GemmParams p, int ntm,
                                                           int ntn, int ntypes, bool vec) {
  constexpr int TM = TL::TM, TN = TL::TN, WTM = TL::WTM, WTN = TL::WTN, MI = TL::MI, NJ = TL::NJ;
  constexpr int NQA = TL::NQA, NQW = TL::NQW, LPS = TL::LPS, STAGE = TL::STAGE;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int tid = threadIdx.x, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w / WGN, wn = w % WGN;
  // accumulators hold C^T for the plain outputs (staged through LDS), C for the residual form
  constexpr bool TR = EPI == 0;
  // byte strides and K in bytes (the parameter block counts elements)
  constexpr int ES = AT == A_I8 ? 1 : 2;
  const int astr = p.a_stride * ES, wstr = p.w_stride * ES;

  // tile order: XCD-contiguous ranges (workgroup b runs on XCD b % 8), then bands of SW row tiles
  const int nb = gridDim.x, b = blockIdx.x;
  const int per = nb >> 3, rem = nb & 7, xcd = b & 7, loc = b >> 3;
  const int lid = (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + loc;
  const int band = lid / (SW * ntn), in_band = lid - band * SW * ntn;
  const int rows_in_band = min(SW, ntm - band * SW);
  const int mt = band * SW + in_band % rows_in_band, nt = in_band / rows_in_band;
  const int m0 = mt * TM, n0 = nt * TN;

  // staging: 4 A pieces and 4 W pieces of 16 bytes per thread and step; rows >= M (N) read as zero
  // (the record counts are wave-uniform; readfirstlane keeps the descriptors in scalar registers)
  const int reca = __builtin_amdgcn_readfirstlane(max(0, min(TM, p.M - m0)) * astr);
  const int recw = __builtin_amdgcn_readfirstlane(max(0, min(TN, p.N - n0)) * wstr);
  const __amdgpu_buffer_rsrc_t ra =
      __builtin_amdgcn_make_buffer_rsrc((void *)(A + (size_t)m0 * astr), (short)0, reca, 0x00020000);
  const __amdgpu_buffer_rsrc_t rw =
      __builtin_amdgcn_make_buffer_rsrc((void *)(W + (size_t)n0 * wstr), (short)0, recw, 0x00020000);
  const int nk = p.K * ES / KS;
  // staging: a stage is 512 rows of 64 bytes (A rows 0-255, then W rows); one wave load fills 16 rows, lane l
  // the slot l % 4 of row l / 4, with the source piece that the reader's swizzle expects there. Wave w loads
  // rows 32 w .. 32 w + 31 of A and of W. Steps past the last read zero (offset 2^31, beyond the records).
  const unsigned lds0 = (unsigned)(size_t)(__attribute__((address_space(3))) char *)smem;
  const int lrow = lane >> 2, lpiece = (lane & 3) ^ ((lane >> 4) & 3);
  int offa[NQA], offw[NQW];
#pragma unroll
  for (int q = 0; q < NQA; q++) offa[q] = (16 * (NQA * w + q) + lrow) * astr + lpiece * 16;
#pragma unroll
  for (int q = 0; q < NQW; q++) offw[q] = (16 * (NQW * w + q) + lrow) * wstr + lpiece * 16;
  auto dma = [&](int kt) __attribute__((always_inline)) {
    const unsigned st = lds0 + ((unsigned)kt % NST) * STAGE;
    const bool ok = kt < nk;
#pragma unroll
    for (int q = 0; q < NQA; q++)
      dma16(st + (16 * (NQA * w + q)) * KS, ok ? (unsigned)(offa[q] + kt * KS) : 0x80000000u, ra);
#pragma unroll
    for (int q = 0; q < NQW; q++)
      dma16(st + (TM + 16 * (NQW * w + q)) * KS, ok ? (unsigned)(offw[q] + kt * KS) : 0x80000000u, rw);
  };

  AccOf<AT> acc[MI][NJ];
#pragma unroll
  for (int i = 0; i < MI; i++)
#pragma unroll
    for (int j = 0; j < NJ; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0;

  // Operands of a step: 2 A and 4 W pieces for each 32-byte half of the step's K.
  struct Ops {
    i32x4 a[2][MI], w[2][NJ];
  };
  auto read_ops = [&](Ops &o, int kt) __attribute__((always_inline)) {
    const char *sA = smem + ((unsigned)kt % NST) * STAGE, *sW = sA + TM * KS;
#pragma unroll
    for (int c = 0; c < KS / 32; c++) {
#pragma unroll
      for (int i = 0; i < MI; i++) o.a[c][i] = *(const i32x4 *)(sA + swz(WTM * wm + 32 * i + l32, 2 * c + hl));
#pragma unroll
      for (int j = 0; j < NJ; j++) o.w[c][j] = *(const i32x4 *)(sW + swz(WTN * wn + 32 * j + l32, 2 * c + hl));
    }
  };
  // Step kt: its operands are already in registers (cur). Once stage kt + 1 has landed (own loads: vmcnt;
  // everyone's: the barrier, which also completes every wave's reads of stage kt), stage kt is refilled with
  // step kt + NST, and the MFMAs of step kt are interleaved with the reads of step kt + 1's operands (nxt).
  auto step = [&](int kt, const Ops &cur, Ops &nxt) __attribute__((always_inline)) {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"((NST - 2) * LPS) : "memory");
    __syncthreads();
    dma(kt + NST);
    read_ops(nxt, kt + 1);
#pragma unroll
    for (int c = 0; c < KS / 32; c++)
#pragma unroll
      for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++)
          acc[i][j] = TR ? mma<AT>(cur.w[c][j], cur.a[c][i], acc[i][j]) : mma<AT>(cur.a[c][i], cur.w[c][j], acc[i][j]);
    constexpr int NR = 2 * (MI + NJ), NF = 2 * MI * NJ;  // LDS reads and MFMAs of a step
    if constexpr (NF >= NR) {
#pragma unroll
      for (int g = 0; g < NR; g++) {
        __builtin_amdgcn_sched_group_barrier(0x008, NF / NR, 0);  // MFMAs
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);        // one LDS read
      }
      __builtin_amdgcn_sched_group_barrier(0x008, NF - NR * (NF / NR), 0);
    }
  };

#pragma unroll
  for (int s = 0; s < NST; s++) dma(s);
  Ops o0, o1;
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"((NST - 1) * LPS) : "memory");
  __syncthreads();
  read_ops(o0, 0);
  for (int kt = 0; kt < nk; kt += 2) {
    step(kt, o0, o1);
    if (kt + 1 < nk) step(kt + 1, o1, o0);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  if constexpr (EPI == 1) {
    // residual form: accumulator element e of tile (i, j) is C[m][n] with m = WTM wm + 32 i + 8 (e / 4) + 4 hl +
    // e % 4 and n = WTN wn + 32 j + l32 (tile-relative), so each store writes 128 contiguous bytes of two rows.
    // Stores are per wave, without barriers, so a wave's epilogue overlaps the other waves' MFMAs. Per-row values
    // are loaded once (rows past M clamp to the last row and are not stored); the loads of a tile are issued
    // before its stores.
    auto row_of = [&](int i, int e) { return m0 + WTM * wm + 32 * i + 8 * (e >> 2) + 4 * hl + (e & 3); };
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int i = 0; i < MI; i++) {
      float sam[16];
      int goff[16];
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int m = min(row_of(i, e), p.M - 1);
        if constexpr (SM == S_ROW_COL) sam[e] = sa[m];
        // row types past the gate table's rows clamp to its last
        goff[e] = min((int)rtype[m], ntypes - 1) * p.g_stride;
      }
#pragma unroll
      for (int j = 0; j < NJ; j++) {
        const int n = n0 + WTN * wn + 32 * j + l32;
        const bool nok = n < p.N;
        const int nc = min(n, p.N - 1);
        const float swn = SM != S_NONE ? sw[nc] : 1.0f;
        const float bn = HAS_BIAS ? bias[nc] : 0.0f;
        float xv[16], gv[16];
#pragma unroll
        for (int e = 0; e < 16; e++) {
          xv[e] = ((const float *)out)[(size_t)min(row_of(i, e), p.M - 1) * p.c_stride + nc];
          gv[e] = gate[goff[e] + nc];
        }
#pragma unroll
        for (int e = 0; e < 16; e++) {
          const int m = row_of(i, e);
          float v = (float)acc[i][j][e];
          if constexpr (SM == S_ROW_COL) v = v * sam[e] * swn;
          else if constexpr (SM == S_COL) v = v * swn;
          if constexpr (HAS_BIAS) v += bn;
          if (nok && m < p.M) ((float *)out)[(size_t)m * p.c_stride + n] = xv[e] + gv[e] * v;
        }
      }
    }
    return;
  }

  // plain outputs: accumulator element e of tile (i, j) is C[m][n] with m = WTM wm + 32 i + l32 and
  // n = WTN wn + 32 j + 8 (e / 4) + 4 hl + e % 4 (tile-relative). Rows past M and columns past N are not
  // stored; their loads clamp to the last row and column.
  constexpr int OSZ = OT == T_F32 ? 4 : 2;
  float sam[MI];
#pragma unroll
  for (int i = 0; i < MI; i++) sam[i] = SM == S_ROW_COL ? sa[min(m0 + WTM * wm + 32 * i + l32, p.M - 1)] : 1.0f;
  auto value = [&](int i, int j, int e, float swn, float bn) __attribute__((always_inline)) {
    float v = (float)acc[i][j][e];
    if constexpr (SM == S_ROW_COL) v = v * sam[i] * swn;
    else if constexpr (SM == S_COL) v = v * swn;
    if constexpr (HAS_BIAS) v += bn;
    return v;
  };
  auto ld4 = [&](const float *q, int n) __attribute__((always_inline)) {  // q[n .. n + 3], clamped per element
    float4 r;
    if (vec) {
      r = *(const float4 *)(q + n);
    } else {
      r.x = q[min(n, p.N - 1)];
      r.y = q[min(n + 1, p.N - 1)];
      r.z = q[min(n + 2, p.N - 1)];
      r.w = q[min(n + 3, p.N - 1)];
    }
    return r;
  };
  if constexpr (OT != T_F32) {
    // 16-bit outputs: the tile's values into LDS (rows of TN values, 2 TN + 16 bytes apart), then 16-byte row
    // stores
    constexpr int RS = TN * 2 + 16;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NJ; j++)
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int nl = WTN * wn + 32 * j + 8 * q + 4 * hl, n = n0 + nl;
        float4 s4 = {1, 1, 1, 1};
        if constexpr (SM != S_NONE) s4 = ld4(sw, min(n, vec ? p.N - 4 : n));
        float4 b4 = {0, 0, 0, 0};
        if constexpr (HAS_BIAS) b4 = ld4(bias, min(n, vec ? p.N - 4 : n));
        const float sv[4] = {s4.x, s4.y, s4.z, s4.w}, bv[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
        for (int i = 0; i < MI; i++) {
          unsigned short h[4];
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const float v = value(i, j, 4 * q + r, sv[r], bv[r]);
            if constexpr (OT == T_BF16) h[r] = __builtin_bit_cast(unsigned short, (__bf16)v);
            else h[r] = __builtin_bit_cast(unsigned short, (_Float16)v);
          }
          const int ml = WTM * wm + 32 * i + l32;
          *(uint2 *)(smem + ml * RS + nl * 2) = make_uint2(h[0] | (unsigned)h[1] << 16, h[2] | (unsigned)h[3] << 16);
        }
      }
    __syncthreads();
    // TM rows x TN / 8 pieces of 16 bytes, consecutive threads along a row
    constexpr int PPR = TN / 8;
#pragma unroll 4
    for (int c = tid; c < TM * PPR; c += NWG * 64) {
      const int ml = c / PPR, pc = c % PPR, m = m0 + ml, n = n0 + 8 * pc;
      if (m >= p.M || n >= p.N) continue;
      const uint4 d = *(const uint4 *)(smem + ml * RS + pc * 16);
      char *dst = out + ((size_t)m * p.c_stride + n) * 2;
      if (vec) {
        *(uint4 *)dst = d;
      } else {
        const unsigned short *hs = (const unsigned short *)&d;
        for (int r = 0; r < 8 && n + r < p.N; r++) ((unsigned short *)dst)[r] = hs[r];
      }
    }
  } else {
    // float outputs: half a tile at a time (TM / 2 rows of TN values, 4 TN + 16 bytes apart) into LDS, then 16-byte
    // row stores
    constexpr int RS = TN * 4 + 16, HR = TM / 2;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int h = 0; h < 2; h++) {
      __syncthreads();
      if (WTM * wm / HR == h) {
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
          for (int q = 0; q < 4; q++) {
            const int nl = WTN * wn + 32 * j + 8 * q + 4 * hl, n = n0 + nl;
            float4 s4 = {1, 1, 1, 1};
        if constexpr (SM != S_NONE) s4 = ld4(sw, min(n, vec ? p.N - 4 : n));
            float4 b4 = {0, 0, 0, 0};
            if constexpr (HAS_BIAS) b4 = ld4(bias, min(n, vec ? p.N - 4 : n));
            const float sv[4] = {s4.x, s4.y, s4.z, s4.w}, bv[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
            for (int i = 0; i < MI; i++) {
              float o[4];
#pragma unroll
              for (int r = 0; r < 4; r++) o[r] = value(i, j, 4 * q + r, sv[r], bv[r]);
              const int ml = WTM * wm + 32 * i + l32 - HR * h;
              *(float4 *)(smem + ml * RS + nl * 4) = make_float4(o[0], o[1], o[2], o[3]);
            }
          }
      }
      __syncthreads();
      // 128 rows x 64 pieces of 16 bytes, 16 per thread (rows ml0 + 8 k), consecutive threads along a row;
      constexpr int PPR = TN / 4;  // 16-byte pieces per row
      const int pc = tid % PPR, n = n0 + 4 * pc;
#pragma unroll 4
      for (int ml = tid / PPR; ml < HR; ml += NWG * 64 / PPR) {
        const int m = m0 + HR * h + ml;
        if (m >= p.M || n >= p.N) continue;
        const float4 o = *(const float4 *)(smem + ml * RS + pc * 16);
        float *dst = (float *)out + (size_t)m * p.c_stride + n;
        if (vec) {
          *(float4 *)dst = o;
        } else {
          const float ov[4] = {o.x, o.y, o.z, o.w};
          for (int r = 0; r < 4 && n + r < p.N; r++) dst[r] = ov[r];
        }
      }
    }
  }
}

// h8 weights: the int8 codes widened to half (exact) into a dense [N][K] buffer, which the half kernel reads
__global__ __launch_bounds__(256) void widen_i8_f16(const signed char *__restrict__ q, _Float16 *__restrict__ out,
                                                    int N, int K, int q_stride) {
  const size_t n = blockIdx.y, k = ((size_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if ((int)n >= N || k >= (size_t)K) return;
  typedef signed char c8 __attribute__((ext_vector_type(8)));
  const c8 v = *(const c8 *)(q + n * q_stride + k);
  f16x8 h;
#pragma unroll
  for (int i = 0; i < 8; i++) h[i] = (_Float16)v[i];
  *(f16x8 *)(out + n * K + k) = h;
}

// Formats: WFMT 1 (q8: int8 A and W, sa[m] sw[n]), 4 (f16: half A and W), 5 (bf16), 6 (h8: half A, int8 W with
// sw[n]; W widened to half first).
template <int OT, int EPI, bool HAS_BIAS, int WFMT>
int launch_gemm(const Pipeline &pl, const Exec &ex, const Arg *a, int nargs, const void *params,
                uint32_t params_len, std::string *err) {
  (void)pl;
  constexpr int AT = WFMT == 1 ? A_I8 : WFMT == 5 ? A_BF16 : A_F16;
  constexpr int SM = WFMT == 1 ? S_ROW_COL : WFMT == 6 ? S_COL : S_NONE;
  constexpr int ES = AT == A_I8 ? 1 : 2;             // bytes per A element
  constexpr int WES = WFMT == 1 || WFMT == 6 ? 1 : 2;  // bytes per W element as given
  if (params_len != sizeof(GemmParams)) {
    *err = "parameter block of " + std::to_string(params_len) + " bytes, expected " +
           std::to_string(sizeof(GemmParams));
    return -1;
  }
  GemmParams p;
  memcpy(&p, params, sizeof p);
  constexpr int KE = KS / ES;  // K elements per step
  if (p.M < 0 || p.N < 1 || p.K < KE || p.K % KE || p.a_stride < p.K || p.w_stride < p.K || p.c_stride < p.N ||
      (p.a_stride * ES) % 16 || (p.w_stride * WES) % (WFMT == 6 ? 8 : 16)) {
    *err = "bad shape: M " + std::to_string(p.M) + " N " + std::to_string(p.N) + " K " + std::to_string(p.K) +
           " (a multiple of " + std::to_string(KE) + ") a_stride " + std::to_string(p.a_stride) + " w_stride " +
           std::to_string(p.w_stride) + " (16-byte rows) c_stride " + std::to_string(p.c_stride);
    return -1;
  }
  if (nargs < (EPI ? 8 : 5)) {
    *err = EPI ? "expected buffers a, w, sw, sa, x, bias, rtype, gate" : "expected buffers a, w, sw, sa, out";
    return -1;
  }
  auto need = [&](int i, uint64_t bytes, const char *what) {
    if (!a[i].ptr) {
      *err = std::string(what) + " is not bound";
      return false;
    }
    if (bytes > a[i].avail) {
      *err = std::string(what) + " needs " + std::to_string(bytes) + " bytes, its buffer holds " +
             std::to_string(a[i].avail);
      return false;
    }
    return true;
  };
  if (p.M == 0) return 0;
  const uint64_t M = p.M, N = p.N;
  constexpr int OSZ = OT == T_F32 ? 4 : 2;
  if (!need(0, ((M - 1) * p.a_stride + p.K) * ES, "a") || !need(1, ((N - 1) * p.w_stride + p.K) * WES, "w") ||
      (SM != S_NONE && !need(2, N * 4, "sw")) || (SM == S_ROW_COL && !need(3, M * 4, "sa")) ||
      !need(4, ((M - 1) * p.c_stride + N) * OSZ, "out") || (HAS_BIAS && !need(5, N * 4, "bias")))
    return -1;
  int ntypes = 1;
  if (EPI) {
    if (!need(6, M, "rtype") || !need(7, N * 4, "gate")) return -1;
    if (p.g_stride < p.N) {
      *err = "g_stride " + std::to_string(p.g_stride) + " smaller than N";
      return -1;
    }
    // rows of the gate table the buffer holds; a row type past them uses the last (the types are data)
    ntypes = (int)std::min<uint64_t>(256, (a[7].avail / 4 - N) / p.g_stride + 1);
  }
  for (int i : {0, 1})
    if ((uintptr_t)a[i].ptr % 16) {
      *err = std::string(i ? "w" : "a") + " must be 16-byte aligned";
      return -1;
    }
  const void *wptr = a[1].ptr;
  if constexpr (WFMT == 6) {
    // the widened weights go to the stream's scratch buffer; the product reads them with a dense row stride
    const size_t wbytes = (size_t)N * p.K * 2;
    if (wbytes > ex.ws_bytes) {
      *err = "the widened h8 weights need " + std::to_string(wbytes) + " bytes of scratch, " +
             std::to_string(ex.ws_bytes) + " are reserved (h3_reserve_workspace)";
      return -1;
    }
    _Float16 *wh = (_Float16 *)ex.ws;
    hipLaunchKernelGGL(widen_i8_f16, dim3((unsigned)((p.K / 8 + 255) / 256), (unsigned)N), dim3(256), 0, ex.stream,
                       (const signed char *)a[1].ptr, wh, p.N, p.K, p.w_stride);
    wptr = wh;
    p.w_stride = p.K;
  }
  // 16-byte vector access to the output (and the column vectors) when alignment and N allow it
  constexpr int VE = 16 / OSZ;
  auto al16 = [](const void *q) { return (uintptr_t)q % 16 == 0; };
  const bool vec = al16(a[4].ptr) && (p.c_stride * OSZ) % 16 == 0 && p.N % VE == 0 &&
                   (SM == S_NONE || al16(a[2].ptr)) && (!HAS_BIAS || al16(a[5].ptr)) &&
                   (!EPI || (al16(a[7].ptr) && p.g_stride % 4 == 0));
  // One grid of 256 x 256 tiles; when its last round of tiles would leave more than half the CUs idle, the
  // trailing rows of tiles go to a second launch of 128 x 128 tiles (the same kernel on the sub-problem of those
  // rows: A, sa, rtype and the output offset by the first row), if that shortens the estimated time (a small
  // tile taken as 0.45 of a big one's time).
  auto launch = [&](auto tl, int row0, int rows) -> int {
    using TL = decltype(tl);
    auto kern = gemm_kernel<OT, EPI, HAS_BIAS, AT, SM, TL>;
    constexpr int LDS_BYTES = TL::template lds_bytes<OT>();
    static bool attr_set = false;  // one per tile configuration
    if (!attr_set) {
      hipError_t e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, LDS_BYTES);
      if (e != hipSuccess) {
        *err = std::string("hipFuncSetAttribute: ") + hipGetErrorString(e);
        return -1;
      }
      attr_set = true;
    }
    GemmParams q = p;
    q.M = rows;
    const int ntm = (rows + TL::TM - 1) / TL::TM, ntn = (p.N + TL::TN - 1) / TL::TN;
    const size_t r0 = (size_t)row0;
    hipLaunchKernelGGL(kern, dim3((unsigned)(ntm * ntn)), dim3(NWG * 64), LDS_BYTES, ex.stream,
                       (const char *)a[0].ptr + r0 * p.a_stride * ES, (const char *)wptr,
                       SM != S_NONE ? (const float *)a[2].ptr : nullptr,
                       SM == S_ROW_COL ? (const float *)a[3].ptr + r0 : nullptr, a[4].ptr + r0 * p.c_stride * OSZ,
                       HAS_BIAS ? (const float *)a[5].ptr : nullptr,
                       EPI ? (const unsigned char *)a[6].ptr + r0 : nullptr, EPI ? (const float *)a[7].ptr : nullptr,
                       q, ntm, ntn, ntypes, vec);
    return 0;
  };
  constexpr int BT = TileBig::TM, ST = TileSmall::TM;
  const int ntm = (p.M + BT - 1) / BT, ntn = (p.N + TileBig::TN - 1) / TileBig::TN;
  const int cus = cu_count();
  int main_rows = p.M;
  if (cus > 0) {
    const long nt = (long)ntm * ntn, R = nt % cus;
    const int tr = (int)((R + ntn - 1) / ntn);  // trailing rows of tiles that hold the last round's tiles
    if (R > 0 && 2 * R <= cus && tr < ntm) {
      const int mrows = (ntm - tr) * BT;
      const long small = (long)((p.M - mrows + ST - 1) / ST) * ((p.N + ST - 1) / ST);
      const double t_split = (double)(((long)(ntm - tr) * ntn + cus - 1) / cus) + 0.45 * ((small + cus - 1) / cus);
      if (t_split < (double)((nt + cus - 1) / cus)) main_rows = mrows;
    }
  }
  if (launch(TileBig{}, 0, main_rows)) return -1;
  if (main_rows < p.M && launch(TileSmall{}, main_rows, p.M - main_rows)) return -1;
  return 0;
}

template <int WFMT>
LaunchFn pick(int epi, int ot, bool bias) {
  if (epi) return bias ? launch_gemm<T_F32, 1, true, WFMT> : launch_gemm<T_F32, 1, false, WFMT>;
  if (ot == T_BF16) return bias ? launch_gemm<T_BF16, 0, true, WFMT> : launch_gemm<T_BF16, 0, false, WFMT>;
  if (ot == T_F16) return bias ? launch_gemm<T_F16, 0, true, WFMT> : launch_gemm<T_F16, 0, false, WFMT>;
  return bias ? launch_gemm<T_F32, 0, true, WFMT> : launch_gemm<T_F32, 0, false, WFMT>;
}

}  // namespace

// Macros (those of h3metal/ops.py:161-164): WFMT (1 q8, 4 f16, 5 bf16, 6 h8), EPI (0 or 1), OUT_T (half | bfloat |
// float; float for EPI 1), HAS_BIAS. The reference's tile and layout choices TM, TN, NSG, G, SWZ, FAST_LAYOUT
// are accepted and unused (this kernel's tiles are its own); LORA must be 0.
bool make_gemm(const std::string &fn, const Macros &m, Pipeline *pl, std::string *err) {
  if (fn != "gemm") {
    *err = "unknown function (have: gemm)";
    return false;
  }
  int wfmt, epi, hb, lora, dummy;
  if (!macro_int(m, "WFMT", 1, &wfmt, err) || !macro_int(m, "EPI", 0, &epi, err) ||
      !macro_int(m, "HAS_BIAS", 0, &hb, err) || !macro_int(m, "LORA", 0, &lora, err))
    return false;
  for (const char *k : {"TM", "TN", "NSG", "G", "SWZ", "FAST_LAYOUT"})
    if (!macro_int(m, k, 0, &dummy, err)) return false;
  for (auto &kv : m) {
    static const char *known[] = {"WFMT", "EPI", "OUT_T", "HAS_BIAS", "LORA", "TM", "TN", "NSG", "G", "SWZ",
                                  "FAST_LAYOUT"};
    bool ok = false;
    for (const char *k : known) ok = ok || kv.first == k;
    if (!ok) {
      *err = "unknown macro " + kv.first;
      return false;
    }
  }
  if (wfmt != 1 && wfmt != 4 && wfmt != 5 && wfmt != 6) {
    *err = "weight format " + std::to_string(wfmt) + " not built (WFMT 1 q8, 4 f16, 5 bf16, 6 h8)";
    return false;
  }
  if (lora) {
    *err = "low-rank (LoRA) terms are not built";
    return false;
  }
  if (epi != 0 && epi != 1) {
    *err = "EPI must be 0 or 1";
    return false;
  }
  const std::string t = macro_str(m, "OUT_T", epi ? "float" : "half");
  int ot = t == "bfloat" || t == "bf16" ? T_BF16 : t == "half" || t == "f16" ? T_F16 : t == "float" || t == "f32" ? T_F32 : -1;
  if (ot < 0 || (epi == 1 && ot != T_F32)) {
    *err = "OUT_T must be half|bfloat|float (float with EPI 1)";
    return false;
  }
  pl->launch = wfmt == 1 ? pick<1>(epi, ot, hb != 0)
               : wfmt == 4 ? pick<4>(epi, ot, hb != 0)
               : wfmt == 5 ? pick<5>(epi, ot, hb != 0)
                           : pick<6>(epi, ot, hb != 0);
  pl->threads = NWG * 64;
  return true;
}

}  // namespace h3
