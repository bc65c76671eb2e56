// Pieces shared by the attention kernels (attention.hip, attention_wave.hip): vector types, MFMA wrappers,
// the LDS layouts of K and V, output stores, the tail-split description and its merge kernel.
#pragma once

#include "h3hip_internal.h"

#include <cfloat>
#include <cmath>
#include <string>
#include <type_traits>

namespace h3 {

enum { T_I8 = 0, T_BF16 = 1, T_F16 = 2, T_F32 = 3 };
constexpr int BK = 64;  // keys per LDS block

// Tail split: when the last round of workgroups would leave CUs idle, its tiles (the last tiles in tile order)
// are cut along the keys into `s` chunks of `cb` key blocks each, one workgroup per chunk. A chunk writes its
// unnormalised partial state (O, running maximum m, row sum l) to `ws`, row stride DG + 4 floats (O at 0,
// m at DG, l at DG + 1), and attention_merge combines the chunks of a tile.
struct Split {
  int nfull;  // workgroups that run whole tiles (tiles 0 .. nfull-1)
  int s;      // chunks per split tile (0: no split)
  int cb;     // key blocks per chunk
  float *ws;  // partial states: [unit][BQ rows][DG + 4]
  int rnd;    // compute units per XCD (workgroups per XCD and round; 0: unknown)
};

// The wave-pipelined kernel (attention_wave.hip): launches it (and the merge of a tail split) for D = 128 without
// a causal mask. qkt, vt, ot: T_I8 / T_BF16 / T_F16 / T_F32 codes; `dump` (the scores hook) also writes the raw
// score accumulators to `dump` [H][Lq][L]. Returns 0, or -1 with a message.
#ifndef WAVE_NU
#define WAVE_NU 2
#endif
constexpr int WAVE_BQ = 128 * WAVE_NU;  // query rows per workgroup of the wave-pipelined kernel (32 WAVE_NU per wave)
constexpr int WAVE_THREADS = 256;       // its workgroup: 4 waves, one per SIMD
int launch_attention_wave(int qkt, int vt, int ot, bool dump, const Exec &ex, const Arg *args, const AttnParams &p,
                          int nqb, const Split &sp, std::string *err);

namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));



template <int T> struct Vec8;
template <> struct Vec8<T_BF16> { using type = bf16x8; using pair = bf16x2; using elem = __bf16; };
template <> struct Vec8<T_F16> { using type = f16x8; using pair = f16x2; using elem = _Float16; };

// 32x32 score product with a 16-byte A and B operand per lane.
template <int QKT>
__device__ __forceinline__ auto mma_qk(i32x4 a, i32x4 b, typename std::conditional<QKT == T_I8, i32x16, f32x16>::type c) {
  if constexpr (QKT == T_I8) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
  } else if constexpr (QKT == T_BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  }
}

template <int VT>
__device__ __forceinline__ f32x16 mma_pv(i16x8 a, typename Vec8<VT>::type b, f32x16 c) {
  if constexpr (VT == T_BF16) return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), b, c, 0, 0, 0);
  else return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), b, c, 0, 0, 0);
}

// Sum of a packed pair plus an accumulator (v_dot2_f32_{bf16,f16} with (1, 1)).
template <int VT>
__device__ __forceinline__ float sum2(typename Vec8<VT>::pair p, float acc) {
  if constexpr (VT == T_BF16) return __builtin_amdgcn_fdot2_f32_bf16(p, bf16x2{(__bf16)1.0f, (__bf16)1.0f}, acc, false);
  else return __builtin_amdgcn_fdot2(p, f16x2{(_Float16)1.0f, (_Float16)1.0f}, acc, false);
}

__device__ __forceinline__ i16x4 lds_tr16(const char *p) {
  typedef __attribute__((address_space(3))) i16x4 *LP;
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((LP)p);
}

// LDS on gfx950 serves a 16-byte read 16 lanes at a time from 64 four-byte banks (256 bytes per pass).
// K rows (RB bytes, NP 16-byte pieces) are read 16 lanes = 16 distinct rows at a time: piece p of row `key`
// is stored at p ^ ((key / (256 / RB)) % NP), so the 16 rows of a pass occupy distinct (bank half, piece)
// slots. (For 128-byte rows: 2 rows per 256 bytes and 8 pieces each; for 256-byte rows: 16 pieces.)
template <int RB, int NP>
__device__ __forceinline__ int kswz(int key) {
  return (key / (256 / RB)) % NP;
}

// Byte offset of 16-byte piece pc of V row `key` (rows of D bf16/f16). A transposing read covers 4 rows x 32
// bytes per 16-lane group, two groups (channels D0 and D0 + 16) per pass: 32-byte unit u of the row is stored at
// u ^ 2 ((key % 4) / R), R = rows per 256 bytes, which puts the two groups in disjoint bank halves and the
// four rows of each group in distinct banks.
template <int D>
__device__ __forceinline__ int voff(int key, int pc) {
  constexpr int R = 256 / (D * 2) > 0 ? 256 / (D * 2) : 1;
  const int u = (pc >> 1) ^ (2 * ((key & 3) / R));
  return key * (D * 2) + u * 32 + (pc & 1) * 16;
}

template <int OT>
__device__ __forceinline__ void store4(char *dst, float a, float b, float c, float d) {
  if constexpr (OT == T_F32) {
    *(f32x4 *)dst = f32x4{a, b, c, d};
  } else if constexpr (OT == T_BF16) {
    typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
    *(bf16x4 *)dst = bf16x4{(__bf16)a, (__bf16)b, (__bf16)c, (__bf16)d};
  } else {
    typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
    *(f16x4 *)dst = f16x4{(_Float16)a, (_Float16)b, (_Float16)c, (_Float16)d};
  }
}




// Combines the chunks of the split tiles: m* = max_c m_c, w_c = 2^(m_c - m*), O = sum_c w_c O_c / sum_c w_c l_c
// (the online-softmax merge), written like the attention epilogue. One wave per query row, 4 rows per workgroup.
template <int DG, int OT, int BQ>
__global__ __launch_bounds__(256) void attention_merge(const float *__restrict__ ws, char *__restrict__ O, AttnParams p,
                                                       int nqb, int nfull, int s) {
  constexpr int PER = (DG + 63) / 64;  // channels per lane
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int tr = row / BQ, r = row - tr * BQ;
  const int tile = nfull + tr;
  const int h = tile / nqb, qb = tile - h * nqb;
  const int q = qb * BQ + r;
  if (q >= p.Lq) return;
  const float *w0 = ws + ((size_t)tr * s * BQ + r) * (DG + 4);
  const size_t ustride = (size_t)BQ * (DG + 4);
  float mx = -INFINITY;
#pragma unroll 4
  for (int c = 0; c < s; c++) mx = fmaxf(mx, w0[c * ustride + DG]);
  // lane l holds PER contiguous channels from PER l (one 4- or 8-byte load per chunk; the loops unrolled so that
  // the loads of several chunks are in flight at once)
  static_assert(PER <= 2 && DG % PER == 0, "one or two channels per lane");
  const int d0 = PER * lane;
  const bool dok = d0 < DG;
  float lsum = 0.0f, acc[2] = {0.0f, 0.0f};
#pragma unroll 4
  for (int c = 0; c < s; c++) {
    const float *wr = w0 + c * ustride;
    const float mc = wr[DG];
    const float wt = mc == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mc - mx);
    lsum += wt * wr[DG + 1];
    if (dok) {
      if constexpr (PER == 2) {
        const float2 v = *(const float2 *)(wr + d0);
        acc[0] += wt * v.x;
        acc[1] += wt * v.y;
      } else {
        acc[0] += wt * wr[d0];
      }
    }
  }
  const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
  constexpr int OSZ = OT == T_F32 ? 4 : 2;
  const int seq = h / p.seq_heads;
  char *orow = O + (((size_t)seq * p.seq_rows + q) * p.o_stride + (size_t)(h - seq * p.seq_heads) * DG) * OSZ;
  if (dok) {
    const float v0 = acc[0] * inv, v1 = acc[1] * inv;
    if constexpr (PER == 1) {
      if constexpr (OT == T_F32) *(float *)(orow + d0 * 4) = v0;
      else if constexpr (OT == T_BF16) *(__bf16 *)(orow + d0 * 2) = (__bf16)v0;
      else *(_Float16 *)(orow + d0 * 2) = (_Float16)v0;
    } else if constexpr (OT == T_F32) {
      *(float2 *)(orow + d0 * 4) = make_float2(v0, v1);
    } else if constexpr (OT == T_BF16) {
      *(bf16x2 *)(orow + d0 * 2) = bf16x2{(__bf16)v0, (__bf16)v1};
    } else {
      *(f16x2 *)(orow + d0 * 2) = f16x2{(_Float16)v0, (_Float16)v1};
    }
  }
}

}  // namespace

}  // namespace h3
