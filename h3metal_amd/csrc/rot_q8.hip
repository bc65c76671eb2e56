// Row rotation + int8 for gfx950: the consumer of the attention output (and of
// SwiGLU outputs) in front of the int8 projections.
//
// Semantics of the reference kernel rot_q8 (kernels/ops.metal:272-334, helpers
// :19-47, parameters kernels/params.h:25-29, launcher h3metal/ops.py:214-222):
//  * Row m of the input starts at element m * x_stride; mode 1 (swiglu) reads
//    values from columns 0 .. D-1 and gates from D .. 2D-1 and uses
//    value * (gate / (1 + exp(-gate))) (:270, :291-292).
//  * Every 256-column block is multiplied by the 256-point Walsh-Hadamard
//    matrix over 16 (orthonormal, no sign flips): butterfly stages over the
//    column bits in increasing order, each (a + b, a - b) with a the lower
//    column, then * 0.0625 (:19-47).
//  * One scale per row: amax over the whole row, scale = amax > 0 ? amax / 127
//    : 1, code = rint(v * (1 / scale)) (:304-327); sa[m] = scale.
//  * OUT_HR: the rotated row in half precision instead (no scale) (:297-306).
// Every floating-point step is one IEEE-rounded operation in that order (the
// file is compiled without FMA contraction; division is correctly rounded), so
// a float32 restatement reproduces codes and scales bit for bit (the exp of the
// swiglu gate excepted: library exp implementations differ in the last bit).
//
// gfx950 layout: one workgroup of 256 threads per row. Half wave hw (0..7) owns
// blocks hw, hw + 8, ...; lane l of a half holds columns 8l .. 8l+7 of a block,
// so a half wave loads and stores each block as one contiguous run, the three
// in-lane butterfly stages are register work and the five cross-lane stages
// are DPP / ds_swizzle exchanges. All of a row's loads are issued before the
// first block is transformed (the row stays in registers until its amax is
// known); the per-half maxima meet in LDS. The kernel is HBM-bound.
#include "h3hip_internal.h"

#include <cmath>
#include <cstring>

namespace h3 {
namespace {

enum { T_BF16 = 1, T_F16 = 2, T_F32 = 3 };

template <int T> struct Elem;
template <> struct Elem<T_BF16> { using type = __bf16; };
template <> struct Elem<T_F16> { using type = _Float16; };
template <> struct Elem<T_F32> { using type = float; };

template <int N, typename E> struct VecOf { typedef E type __attribute__((ext_vector_type(N))); };

constexpr int RB = 256;  // rotation block

template <int IN_T, bool SWIGLU, bool OUT_HR, int MAXB>
__global__ __launch_bounds__(256) void rot_q8_kernel(const char *__restrict__ in, char *__restrict__ out,
                                                      float *__restrict__ sa, RotQParams p) {
  using IE = typename Elem<IN_T>::type;
  typedef typename VecOf<8, IE>::type IV;
  __shared__ float red[8];
  const int lane = threadIdx.x & 63, l32 = lane & 31;
  const int hw = (threadIdx.x >> 6) * 2 + (lane >> 5);
  const int m = blockIdx.x;
  const int nb = p.D / RB;
  const IE *row = (const IE *)in + (size_t)m * p.x_stride;

  IV xv[MAXB], xg[SWIGLU ? MAXB : 1];
#pragma unroll
  for (int b = 0; b < MAXB; b++) {
    const int blk = hw + 8 * b;
    if (blk < nb) {
      xv[b] = *(const IV *)(row + blk * RB + l32 * 8);
      if constexpr (SWIGLU) xg[b] = *(const IV *)(row + p.D + blk * RB + l32 * 8);
    }
  }
  float v[MAXB][8];
  float amax = 0.0f;
#pragma unroll
  for (int b = 0; b < MAXB; b++) {
    const int blk = hw + 8 * b;
    if (blk >= nb) continue;  // uniform over the half wave
#pragma unroll
    for (int i = 0; i < 8; i++) {
      float val = (float)xv[b][i];
      if constexpr (SWIGLU) {
        const float g = (float)xg[b][i];
        val = val * (g / (1.0f + expf(-g)));
      }
      v[b][i] = val;
    }
    // columns 8 l32 + i: bits 0-2 in the lane, bits 3-7 across lanes
#pragma unroll
    for (int s = 1; s < 8; s <<= 1)
#pragma unroll
      for (int i = 0; i < 8; i++)
        if (!(i & s)) {
          const float a = v[b][i], c = v[b][i + s];
          v[b][i] = a + c;
          v[b][i + s] = a - c;
        }
    // across lanes (column bits 3-7): the lower column becomes a + b, the upper a - b; each lane ends with its
    // values times (-1)^popcount(l32), folded into the final 1/16 (hadamard_lane_stage)
    auto stage = [&](auto ls_const) {
      constexpr int LS = decltype(ls_const)::value;
      hadamard_lane_stage<LS>(v[b], (l32 & LS) ? -1.0f : 1.0f);
    };
    stage(std::integral_constant<int, 1>{});
    stage(std::integral_constant<int, 2>{});
    stage(std::integral_constant<int, 4>{});
    stage(std::integral_constant<int, 8>{});
    stage(std::integral_constant<int, 16>{});
    const float sc = (__builtin_popcount(l32) & 1) ? -0.0625f : 0.0625f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      v[b][i] *= sc;
      amax = fmaxf(amax, fabsf(v[b][i]));
    }
  }
  if constexpr (OUT_HR) {
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    _Float16 *o = (_Float16 *)out + (size_t)m * p.D;
#pragma unroll
    for (int b = 0; b < MAXB; b++) {
      const int blk = hw + 8 * b;
      if (blk < nb) {
        h8 hv;
#pragma unroll
        for (int i = 0; i < 8; i++) hv[i] = (_Float16)v[b][i];
        *(h8 *)(o + blk * RB + l32 * 8) = hv;
      }
    }
    return;
  } else {
    amax = fmaxf(amax, xshfl<16>(amax));
    amax = fmaxf(amax, xshfl<8>(amax));
    amax = fmaxf(amax, xshfl<4>(amax));
    amax = fmaxf(amax, xshfl<2>(amax));
    amax = fmaxf(amax, xshfl<1>(amax));
    if (l32 == 0) red[hw] = amax;
    __syncthreads();
    amax = red[0];
#pragma unroll
    for (int i = 1; i < 8; i++) amax = fmaxf(amax, red[i]);
    const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    const float rs = 1.0f / scale;
    typedef signed char c8 __attribute__((ext_vector_type(8)));
    char *o = out + (size_t)m * p.D;
#pragma unroll
    for (int b = 0; b < MAXB; b++) {
      const int blk = hw + 8 * b;
      if (blk < nb) {
        c8 cv;
#pragma unroll
        for (int i = 0; i < 8; i++) cv[i] = (signed char)(int)rintf(v[b][i] * rs);
        *(c8 *)(o + blk * RB + l32 * 8) = cv;
      }
    }
    if (threadIdx.x == 0) sa[m] = scale;
  }
}

int esize(int t) { return t == T_F32 ? 4 : 2; }

template <int IN_T, bool OUT_HR, int MAXB>
int launch_rot(const Pipeline &pl, const Exec &ex, const Arg *a, int nargs, const void *params,
               uint32_t params_len, std::string *err) {
  (void)pl;
  if (params_len != sizeof(RotQParams)) {
    *err = "parameter block of " + std::to_string(params_len) + " bytes, expected " +
           std::to_string(sizeof(RotQParams));
    return -1;
  }
  RotQParams p;
  memcpy(&p, params, sizeof p);
  const int width = p.mode ? 2 * p.D : p.D;
  if (p.M < 0 || p.D < RB || p.D % RB || (p.mode != 0 && p.mode != 1) || p.x_stride < width) {
    *err = "bad shape: M " + std::to_string(p.M) + " D " + std::to_string(p.D) + " (a positive multiple of 256)" +
           " x_stride " + std::to_string(p.x_stride) + " mode " + std::to_string(p.mode);
    return -1;
  }
  if (p.D / RB > 8 * MAXB) {
    *err = "D " + std::to_string(p.D) + " exceeds this specialisation's " + std::to_string(8 * MAXB * RB) +
           " columns";
    return -1;
  }
  const int need = OUT_HR ? 2 : 3;
  if (nargs < need || !a[0].ptr || !a[1].ptr || (!OUT_HR && !a[2].ptr)) {
    *err = OUT_HR ? "expected buffers x, out" : "expected buffers x, out, sa";
    return -1;
  }
  auto fits = [&](int i, uint64_t bytes, const char *what) {
    if (bytes > a[i].avail) {
      *err = std::string(what) + " needs " + std::to_string(bytes) + " bytes, its buffer holds " +
             std::to_string(a[i].avail);
      return false;
    }
    return true;
  };
  if (p.M == 0) return 0;
  const uint64_t in_bytes = ((uint64_t)(p.M - 1) * p.x_stride + width) * esize(IN_T);
  if (!fits(0, in_bytes, "x") || !fits(1, (uint64_t)p.M * p.D * (OUT_HR ? 2 : 1), "out") ||
      (!OUT_HR && !fits(2, (uint64_t)p.M * 4, "sa")))
    return -1;
  if (p.mode)
    hipLaunchKernelGGL((rot_q8_kernel<IN_T, true, OUT_HR, MAXB>), dim3((unsigned)p.M), dim3(256), 0, ex.stream,
                       a[0].ptr, a[1].ptr, OUT_HR ? nullptr : (float *)a[2].ptr, p);
  else
    hipLaunchKernelGGL((rot_q8_kernel<IN_T, false, OUT_HR, MAXB>), dim3((unsigned)p.M), dim3(256), 0, ex.stream,
                       a[0].ptr, a[1].ptr, OUT_HR ? nullptr : (float *)a[2].ptr, p);
  return 0;
}

template <int IN_T, bool OUT_HR>
LaunchFn pick_maxb(int maxb) {
  if (maxb <= 1) return launch_rot<IN_T, OUT_HR, 1>;
  if (maxb <= 2) return launch_rot<IN_T, OUT_HR, 2>;
  if (maxb <= 4) return launch_rot<IN_T, OUT_HR, 4>;
  if (maxb <= 8) return launch_rot<IN_T, OUT_HR, 8>;
  return launch_rot<IN_T, OUT_HR, 16>;
}

}  // namespace

// Macros (those of h3metal/ops.py:220): IN_T (half | bfloat | float), OUT_HR, and NSG / MAXB, the reference's
// SIMD-groups per threadgroup and rotation blocks per SIMD-group. NSG * MAXB * 256 bounds the row length as in
// the reference; here a row's blocks are spread over 8 half waves, so MAXB selects the specialisation holding
// ceil(NSG * MAXB / 8) blocks per half wave (rows up to 32768 columns).
bool make_rot_q8(const Macros &m, Pipeline *pl, std::string *err) {
  int nsg, maxb, hr;
  if (!macro_int(m, "NSG", 8, &nsg, err) || !macro_int(m, "MAXB", 3, &maxb, err) ||
      !macro_int(m, "OUT_HR", 0, &hr, err))
    return false;
  for (auto &kv : m) {
    static const char *known[] = {"NSG", "MAXB", "IN_T", "OUT_HR"};
    bool ok = false;
    for (const char *k : known) ok = ok || kv.first == k;
    if (!ok) {
      *err = "unknown macro " + kv.first;
      return false;
    }
  }
  const int blocks = nsg * maxb;
  if (nsg < 1 || maxb < 1 || blocks > 128) {
    *err = "NSG * MAXB must be between 1 and 128 rotation blocks";
    return false;
  }
  const int per = (blocks + 7) / 8;
  const std::string t = macro_str(m, "IN_T", "bfloat");
  LaunchFn f = nullptr;
  if (t == "bfloat" || t == "bf16") f = hr ? pick_maxb<T_BF16, true>(per) : pick_maxb<T_BF16, false>(per);
  else if (t == "half" || t == "f16") f = hr ? pick_maxb<T_F16, true>(per) : pick_maxb<T_F16, false>(per);
  else if (t == "float" || t == "f32") f = hr ? pick_maxb<T_F32, true>(per) : pick_maxb<T_F32, false>(per);
  if (!f) {
    *err = "IN_T must be half|bfloat|float";
    return false;
  }
  pl->launch = f;
  pl->threads = 256;
  return true;
}

}  // namespace h3
