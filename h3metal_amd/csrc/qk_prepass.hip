// Queries/keys pre-pass for attention, fused in one kernel for gfx950:
// per-head RMS norm, rotary embedding, Walsh-Hadamard rotation with fixed
// signs, and per-row int8 quantisation; values are copied through.
//
// Semantics of the reference kernel qk_norm_rope (kernels/ops.metal:365-468,
// parameters :344-349, launcher h3metal/ops.py:225-239):
//  * Input rows hold Hq query heads, then Hk key heads, then Hv value heads of
//    HDIM channels each (a "slot" is one of them); row m is row r = m % seq_len
//    of sequence m / seq_len, whose heads are output heads sq*H .. sq*H + H-1,
//    row r of each (:381, :448).
//  * norm: v = (v * 1/sqrt(sum(v^2)/HDIM + eps)) * w (:394-402).
//  * rot: the first `rot` channels are rotated in pairs (i, i + rot/2) by the
//    row's angle table: v_i c - v_{i+rot/2} s and v_{i+rot/2} c + v_i s (:403-419).
//  * QKROT (int8 outputs only): v_c = -v_c where popcount(c * 0x2545F491) is odd,
//    then a 128-point fast Walsh-Hadamard transform with its butterfly stages in
//    increasing channel-bit order, each (a + b, a - b) with a the lower channel,
//    then a multiply by 1/sqrt(HDIM) (:420-446).
//  * QK8: scale = amax > 0 ? amax / 127 : 1, code = rint(v / scale) (:450-458).
// Every floating-point step is a single IEEE-rounded operation in that order
// (this file is compiled without FMA contraction; division and square root are
// correctly rounded), so a float32 restatement reproduces codes and scales bit
// for bit. The sum of squares is summed per lane, then over the lanes of a
// head with an xor butterfly (halving strides): a fixed order.
//
// gfx950 layout: a head's channels are spread over a group of lanes, PER
// consecutive channels per lane: PER = 8 (16-byte loads of 16-bit rows; 16
// lanes per head at HDIM 128) whenever the rotary pairs (c, c + rot/2) stay
// lane-aligned (rot/2 a multiple of 8), else the reference's HDIM / 32. Every
// cross-lane step stays inside the group and runs on DPP lane patterns at 16
// lanes per slot (ds_swizzle at other shapes; no LDS memory traffic). A workgroup of 256 threads covers 4 waves' groups of slots
// of 8 consecutive rows; each wave issues all 8 rows' loads before processing
// them, so enough bytes are in flight to stream HBM, and a slot's 8 scales are
// stored together. The kernel is HBM-bound: one read of the rows, one write of
// the codes / values.
#include "h3hip_internal.h"

#include <cmath>
#include <cstring>
#include <type_traits>

namespace h3 {
namespace {

enum { T_I8 = 0, T_BF16 = 1, T_F16 = 2, T_F32 = 3 };

template <int T> struct Elem;
template <> struct Elem<T_BF16> { using type = __bf16; };
template <> struct Elem<T_F16> { using type = _Float16; };
template <> struct Elem<T_F32> { using type = float; };

template <int N, typename E> struct VecOf { typedef E type __attribute__((ext_vector_type(N))); };

constexpr int RPW = 8;  // rows per workgroup; each wave walks them with all their loads in flight

template <int HDIM>
constexpr double inv_sqrt_hdim() {
  return HDIM == 128 ? 0.0883883476483184405501055452631 : HDIM == 64 ? 0.125 : 0.1767766952966368811;
}

// PER channels per lane, LPS = HDIM / PER lanes per (row, head) slot, 64 / LPS slots per wave. Workgroup
// (bx, by): rows bx*RPW .. bx*RPW + RPW-1, slots by*SPG .. by*SPG + SPG-1 (SPG = 4 waves' slots). A lane group
// owns one slot and walks the rows; its lane r keeps the scale of row r so that a slot's RPW scales (consecutive
// in memory within a sequence) are stored together after the rows.
template <int HDIM, int PER>
struct PrepassShape {
  static constexpr int LPS = HDIM / PER;     // lanes per slot
  static constexpr int SPG = 4 * 64 / LPS;   // slots per workgroup
  static_assert(LPS >= RPW && LPS <= 32 && (LPS & (LPS - 1)) == 0, "lane group");
};

// Channel groups and lanes. With 16 lanes per slot the group g (channels 8 g .. 8 g + 7) sits in lane
// L(g) = g0 ^ 2 g1 ^ 7 g2 ^ 8 g3 (g_b the bits of g): the partner along group bit 0, 1, 2, 3 is then lane L ^ 1,
// ^ 2, ^ 7, ^ 8 -- all four DPP lane patterns within a 16-lane row (quad_perm, row_half_mirror, row_ror:8), so
// every cross-lane step of the transform and of the reductions is one VALU instruction with no LDS traffic.
// Other lane counts keep g = lane.
template <int LPS>
__device__ __forceinline__ int group_of_lane(int l) {
  if constexpr (LPS != 16) return l;
  const int g2 = (l >> 2) & 1, r = l ^ (7 * g2);
  return (r & 1) | (r & 2) | (g2 << 2) | (r & 8);
}
template <int LPS>
__device__ __forceinline__ int lane_of_group(int g) {
  if constexpr (LPS != 16) return g;
  return (g & 1) ^ (g & 2) ^ (7 * ((g >> 2) & 1)) ^ (g & 8);
}
// the value of the lane whose group differs in group bit B
template <int LPS, int B>
__device__ __forceinline__ float gshfl(float v) {
  if constexpr (LPS == 16 && B == 4)
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, true));
  else return xshfl<B>(v);
}
// one cross-lane Hadamard stage along group bit B (see hadamard_lane_stage for the sign convention)
template <int LPS, int B, int N>
__device__ __forceinline__ void group_stage(float (&v)[N], float c) {
  if constexpr (LPS == 16 && B == 4) {
    H3_DPP_FMAC_STAGE("row_half_mirror row_mask:0xf bank_mask:0xf bound_ctrl:1");
  } else {
    hadamard_lane_stage<B>(v, c);
  }
}

template <int HDIM, int PER, int IN_T, int QK_T, int V_T, bool QKROT>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(const char *__restrict__ in, const float *__restrict__ wq,
                                                            const float *__restrict__ wk,
                                                            const float *__restrict__ cs,
                                                            const float *__restrict__ sn, char *__restrict__ Qo,
                                                            char *__restrict__ Ko, char *__restrict__ Vo,
                                                            float *__restrict__ qsc, float *__restrict__ ksc,
                                                            QkRopeParams p) {
  using SH = PrepassShape<HDIM, PER>;
  constexpr int LPS = SH::LPS;
  using IE = typename Elem<IN_T>::type;
  typedef typename VecOf<PER, IE>::type IV;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int l32 = lane & (LPS - 1);  // lane within the slot's group
  const int gbase = lane & ~(LPS - 1);  // first lane of the group
  const int g = group_of_lane<LPS>(l32);  // this lane's channel group: channels g * PER .. g * PER + PER - 1
  const int slot = blockIdx.y * SH::SPG + w * (64 / LPS) + lane / LPS;
  const int m0 = blockIdx.x * RPW;
  const int nslots = p.Hq + p.Hk + p.Hv;
  if (slot >= nslots) return;  // whole lane groups only; no cross-lane step leaves a group
  const int nr = min(RPW, p.M - m0);
  // outputs are streamed out with nontemporal stores (nothing in this kernel reads them again; measured +6%)
  auto st = [](auto *dst, auto val) { __builtin_nontemporal_store(val, dst); };

  IV xin[RPW];
  {
    const IE *src = (const IE *)in + (size_t)m0 * p.in_stride + (size_t)slot * HDIM + g * PER;
#pragma unroll
    for (int r = 0; r < RPW; r++) xin[r] = *(const IV *)(src + (size_t)min(r, nr - 1) * p.in_stride);
  }
  const bool isqk = slot < p.Hq + p.Hk, isq = slot < p.Hq;
  const int h = isq ? slot : isqk ? slot - p.Hq : slot - p.Hq - p.Hk;
  const int heads = isq ? p.Hq : isqk ? p.Hk : p.Hv;
  auto hrow_of = [&](int m) {
    const int sq = m / p.seq_len, r = m - sq * p.seq_len;
    return ((size_t)sq * heads + h) * p.out_rows + r;
  };
  float keep = 1.0f;  // lane l32 < nr: the scale of row m0 + l32
  // QKROT's fixed signs: channel c = g * PER + i is negated when popcount(c * 0x2545F491) is odd (its sign
  // bit, flipped by an xor; computed once per lane)
  unsigned sbit[PER];
#pragma unroll
  for (int i = 0; i < PER; i++)
    sbit[i] = (__builtin_popcount((unsigned)(g * PER + i) * 0x2545F491u) & 1u) ? 0x80000000u : 0u;

#pragma unroll
  for (int rr = 0; rr < RPW; rr++) {
    if (rr >= nr) break;
    const int m = m0 + rr;
    float v[PER];
#pragma unroll
    for (int i = 0; i < PER; i++) v[i] = (float)xin[rr][i];
    const size_t hrow = hrow_of(m);
    if (isqk) {
      if (p.norm) {
        float ss = v[0] * v[0];
#pragma unroll
        for (int i = 1; i < PER; i++) ss = ss + v[i] * v[i];
        // over the groups in halving strides (the partner of group g is g ^ stride)
        if constexpr (LPS > 16) ss = ss + gshfl<LPS, 16>(ss);
        if constexpr (LPS > 8) ss = ss + gshfl<LPS, 8>(ss);
        ss = ss + gshfl<LPS, 4>(ss);
        ss = ss + gshfl<LPS, 2>(ss);
        ss = ss + gshfl<LPS, 1>(ss);
        const float inv = 1.0f / sqrtf(ss / (float)HDIM + p.eps);
        const float *wv = (isq ? wq : wk) + g * PER;
#pragma unroll
        for (int i = 0; i < PER; i++) v[i] = (v[i] * inv) * wv[i];
      }
      if (p.rot) {
        const int r = m % p.seq_len;
        const int half_rot = p.rot / 2;
        const int lanes = half_rot / PER;  // lanes holding the first half of the rotated channels
        const int src_group = g < lanes ? g + lanes : (g < 2 * lanes ? g - lanes : g);
        float pv[PER];
#pragma unroll
        for (int i = 0; i < PER; i++) pv[i] = __shfl(v[i], gbase + lane_of_group<LPS>(src_group));
        if (g < 2 * lanes) {
          const bool first = g < lanes;
          const int base = (first ? g : g - lanes) * PER;  // pair index of v[0]
          const float *c = cs + (size_t)r * half_rot + base;
          const float *s = sn + (size_t)r * half_rot + base;
#pragma unroll
          for (int i = 0; i < PER; i++) v[i] = first ? v[i] * c[i] - pv[i] * s[i] : v[i] * c[i] + pv[i] * s[i];
        }
      }
      if constexpr (QKROT) {
#pragma unroll
        for (int i = 0; i < PER; i++) v[i] = __builtin_bit_cast(float, __builtin_bit_cast(unsigned, v[i]) ^ sbit[i]);
#pragma unroll
        for (int s = 1; s < PER; s <<= 1) {
#pragma unroll
          for (int i = 0; i < PER; i++) {
            if (!(i & s)) {
              const float a = v[i], b = v[i + s];
              v[i] = a + b;
              v[i + s] = a - b;
            }
          }
        }
        // across lanes: channel c pairs with c ^ (ls * PER), stages in increasing bit order; the lower channel
        // becomes a + b, the upper one a - b (a the lower channel's value); each lane ends with its values
        // times (-1)^popcount(g) (hadamard_lane_stage)
        auto stage = [&](auto ls_const) {
          constexpr int LS = decltype(ls_const)::value;
          group_stage<LPS, LS>(v, (g & LS) ? -1.0f : 1.0f);
        };
        stage(std::integral_constant<int, 1>{});
        stage(std::integral_constant<int, 2>{});
        stage(std::integral_constant<int, 4>{});
        if constexpr (LPS > 8) stage(std::integral_constant<int, 8>{});
        if constexpr (LPS > 16) stage(std::integral_constant<int, 16>{});
        // the sign carried by the lane goes into the final scale (an exact sign change of the same product)
        constexpr float rn = (float)inv_sqrt_hdim<HDIM>();
        const float rns = (__builtin_popcount(g) & 1) ? -rn : rn;
#pragma unroll
        for (int i = 0; i < PER; i++) v[i] *= rns;
      }
      if constexpr (QK_T == T_I8) {
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < PER; i++) amax = fmaxf(amax, fabsf(v[i]));
        if constexpr (LPS > 16) amax = fmaxf(amax, gshfl<LPS, 16>(amax));
        if constexpr (LPS > 8) amax = fmaxf(amax, gshfl<LPS, 8>(amax));
        amax = fmaxf(amax, gshfl<LPS, 4>(amax));
        amax = fmaxf(amax, gshfl<LPS, 2>(amax));
        amax = fmaxf(amax, gshfl<LPS, 1>(amax));
        const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
        const float rs = __builtin_amdgcn_rcpf(scale);  // 1 ulp
        typedef typename VecOf<PER, signed char>::type CV;
        CV codes;
#pragma unroll
        for (int i = 0; i < PER; i++) codes[i] = (signed char)(int)rintf(v[i] * rs);
        // |v / scale| <= 127.5 and rs is within 1 ulp of 1/scale, so v * rs is within 2^-16 + 2^-18 < 2^-15 of
        // the exact quotient: its nearest integer is the quotient's unless it lies within 2^-15 of a
        // half-integer, and then the lanes concerned divide (rare, and exact). A scale whose reciprocal is not
        // a normal float (amax below ~2^-119) divides on every lane.
        bool near_half = !(rs < 0x1p126f);
#pragma unroll
        for (int i = 0; i < PER; i++) {
          const float y = v[i] * rs;
          near_half |= fabsf(y - rintf(y)) > 0.5f - 0x1p-15f;
        }
        if (near_half) {
#pragma unroll
          for (int i = 0; i < PER; i++) codes[i] = (signed char)(int)rintf(v[i] / scale);
        }
        st((CV *)((isq ? Qo : Ko) + hrow * HDIM + g * PER), codes);
        if (l32 == rr) keep = scale;
      } else {
        using OE = typename Elem<QK_T>::type;
        typedef typename VecOf<PER, OE>::type OV;
        OV out;
#pragma unroll
        for (int i = 0; i < PER; i++) out[i] = (OE)v[i];
        st((OV *)((isq ? Qo : Ko) + (hrow * HDIM + g * PER) * sizeof(OE)), out);
      }
    } else {
      using OE = typename Elem<V_T>::type;
      typedef typename VecOf<PER, OE>::type OV;
      if constexpr (V_T == IN_T) {
        st((OV *)(Vo + (hrow * HDIM + g * PER) * sizeof(OE)), xin[rr]);  // same type: a plain copy
      } else {
        OV out;
#pragma unroll
        for (int i = 0; i < PER; i++) out[i] = (OE)v[i];
        st((OV *)(Vo + (hrow * HDIM + g * PER) * sizeof(OE)), out);
      }
    }
  }
  if constexpr (QK_T == T_I8) {
    if (isqk && l32 < nr) (isq ? qsc : ksc)[hrow_of(m0 + l32)] = keep;
  }
}

int esize(int t) { return t == T_I8 ? 1 : t == T_F32 ? 4 : 2; }

template <int HDIM, int IN_T, int QK_T, int V_T, bool QKROT>
int launch_qk(const Pipeline &pl, const Exec &ex, const Arg *a, int nargs, const void *params,
              uint32_t params_len, std::string *err) {
  (void)pl;
  if (params_len != sizeof(QkRopeParams)) {
    *err = "parameter block of " + std::to_string(params_len) + " bytes, expected " +
           std::to_string(sizeof(QkRopeParams));
    return -1;
  }
  QkRopeParams p;
  memcpy(&p, params, sizeof p);
  const int PER = HDIM / 32;
  const int nslots = p.Hq + p.Hk + p.Hv;
  if (p.M < 0 || p.Hq < 0 || p.Hk < 0 || p.Hv < 0 || nslots < 1 || p.seq_len < 1 || p.out_rows < 1 ||
      p.in_stride < nslots * HDIM) {
    *err = "bad shape: M " + std::to_string(p.M) + " heads " + std::to_string(p.Hq) + "/" + std::to_string(p.Hk) +
           "/" + std::to_string(p.Hv) + " in_stride " + std::to_string(p.in_stride) + " seq_len " +
           std::to_string(p.seq_len);
    return -1;
  }
  const int rows = p.M < p.seq_len ? p.M : p.seq_len;  // rows per sequence actually present
  if (rows > p.out_rows) {
    *err = "out_rows " + std::to_string(p.out_rows) + " smaller than the rows of a sequence";
    return -1;
  }
  if (p.rot < 0 || p.rot > HDIM || p.rot % 2 || (p.rot / 2) % PER) {
    *err = "rot " + std::to_string(p.rot) + " must be even, at most HD, and rot/2 a multiple of " +
           std::to_string(PER);
    return -1;
  }
  if (p.norm && !(p.eps >= 0.0f)) {
    *err = "eps must be non-negative";
    return -1;
  }
  if (nargs < 11 && QK_T == T_I8) {
    *err = "int8 outputs need buffers q_scale and k_scale (indices 9, 10)";
    return -1;
  }
  if (nargs < 8) {
    *err = "expected buffers qkv, wq, wk, cos, sin, Q, K, V";
    return -1;
  }
  auto need = [&](int i, uint64_t bytes, const char *what, bool required) {
    if (!required || bytes == 0) return true;
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
  const uint64_t nseq = p.M ? (uint64_t)(p.M - 1) / p.seq_len + 1 : 0;
  const uint64_t in_bytes = p.M ? ((uint64_t)(p.M - 1) * p.in_stride + (uint64_t)nslots * HDIM) * esize(IN_T) : 0;
  // Rows written per output: head-major rows up to (last head) * out_rows + (rows of a sequence). Callers pass
  // views that start inside a head's row block (h3metal/flux2.py:417-426 writes text rows, then image rows at
  // offset r0), so the check is on the extent actually touched, not on heads * out_rows.
  auto extent = [&](int heads) -> uint64_t {
    return heads && nseq ? (nseq * heads - 1) * (uint64_t)p.out_rows + (uint64_t)rows : 0;
  };
  const uint64_t hq = extent(p.Hq), hk = extent(p.Hk), hv = extent(p.Hv);
  const uint64_t tab = (uint64_t)rows * (p.rot / 2) * 4;
  if (!need(0, in_bytes, "qkv", true) || !need(1, HDIM * 4, "wq", p.norm && p.Hq) ||
      !need(2, HDIM * 4, "wk", p.norm && p.Hk) || !need(3, tab, "cos", p.rot > 0 && (p.Hq + p.Hk)) ||
      !need(4, tab, "sin", p.rot > 0 && (p.Hq + p.Hk)) || !need(5, hq * HDIM * esize(QK_T), "Q", p.Hq > 0) ||
      !need(6, hk * HDIM * esize(QK_T), "K", p.Hk > 0) || !need(7, hv * HDIM * esize(V_T), "V", p.Hv > 0))
    return -1;
  if (QK_T == T_I8 && (!need(9, hq * 4, "q_scale", p.Hq > 0) || !need(10, hk * 4, "k_scale", p.Hk > 0))) return -1;
  if (p.M == 0) return 0;
  // 8 channels per lane (16-byte loads for 16-bit inputs) unless the rotary pairs would straddle lanes, then
  // the reference's HDIM / 32
  auto go = [&](auto per_const) {
    constexpr int P = decltype(per_const)::value;
    constexpr int SPG = PrepassShape<HDIM, P>::SPG;
    dim3 grid((unsigned)((p.M + RPW - 1) / RPW), (unsigned)((nslots + SPG - 1) / SPG));
    hipLaunchKernelGGL((qk_norm_rope_kernel<HDIM, P, IN_T, QK_T, V_T, QKROT>), grid, dim3(256), 0, ex.stream, a[0].ptr,
                       (const float *)a[1].ptr, (const float *)a[2].ptr, (const float *)a[3].ptr,
                       (const float *)a[4].ptr, a[5].ptr, a[6].ptr, a[7].ptr,
                       nargs > 9 ? (float *)a[9].ptr : nullptr, nargs > 10 ? (float *)a[10].ptr : nullptr, p);
  };
  if ((p.rot / 2) % 8 == 0) go(std::integral_constant<int, 8>{});
  else go(std::integral_constant<int, HDIM / 32>{});
  return 0;
}

template <int HDIM, int IN_T>
LaunchFn pick_out(int qk_t, int v_t, bool rot, std::string *err) {
  if (qk_t == T_I8) {
    if (v_t == T_BF16) return rot ? launch_qk<HDIM, IN_T, T_I8, T_BF16, true> : launch_qk<HDIM, IN_T, T_I8, T_BF16, false>;
    return rot ? launch_qk<HDIM, IN_T, T_I8, T_F16, true> : launch_qk<HDIM, IN_T, T_I8, T_F16, false>;
  }
  if (rot) {
    *err = "QKROT needs QK8 (int8 outputs)";
    return nullptr;
  }
  if (qk_t == T_BF16)
    return v_t == T_BF16 ? launch_qk<HDIM, IN_T, T_BF16, T_BF16, false> : launch_qk<HDIM, IN_T, T_BF16, T_F16, false>;
  return v_t == T_BF16 ? launch_qk<HDIM, IN_T, T_F16, T_BF16, false> : launch_qk<HDIM, IN_T, T_F16, T_F16, false>;
}

template <int HDIM>
LaunchFn pick_in(int in_t, int qk_t, int v_t, bool rot, std::string *err) {
  switch (in_t) {
    case T_BF16: return pick_out<HDIM, T_BF16>(qk_t, v_t, rot, err);
    case T_F16: return pick_out<HDIM, T_F16>(qk_t, v_t, rot, err);
    default: return pick_out<HDIM, T_F32>(qk_t, v_t, rot, err);
  }
}

int type_of(const std::string &s) {
  if (s == "bfloat" || s == "bf16") return T_BF16;
  if (s == "half" || s == "f16") return T_F16;
  if (s == "float" || s == "f32") return T_F32;
  return -1;
}

}  // namespace

// Specialisation macros: HDIM (64 or 128), IN_T (input: half | bfloat | float),
// QK8 (int8 Q/K + scales), QKROT (rotation; needs QK8), QK_T (Q/K without QK8:
// half | bfloat, default half as in the reference), V_T (half | bfloat, default
// half). NSG (the reference's SIMD-groups per threadgroup) is accepted and unused.
bool make_ops(const std::string &fn, const Macros &m, Pipeline *pl, std::string *err) {
  if (fn == "rot_q8") return make_rot_q8(m, pl, err);
  if (fn != "qk_norm_rope") {
    *err = "unknown function (have: qk_norm_rope, rot_q8)";
    return false;
  }
  int hd, q8, rot, nsg;
  if (!macro_int(m, "HDIM", 128, &hd, err) || !macro_int(m, "QK8", 0, &q8, err) ||
      !macro_int(m, "QKROT", 0, &rot, err) || !macro_int(m, "NSG", 8, &nsg, err))
    return false;
  for (auto &kv : m) {
    static const char *known[] = {"HDIM", "IN_T", "QK8", "QKROT", "QK_T", "V_T", "NSG"};
    bool ok = false;
    for (const char *k : known) ok = ok || kv.first == k;
    if (!ok) {
      *err = "unknown macro " + kv.first;
      return false;
    }
  }
  const int in_t = type_of(macro_str(m, "IN_T", "half"));
  const int qk_t = q8 ? T_I8 : type_of(macro_str(m, "QK_T", "half"));
  const int v_t = type_of(macro_str(m, "V_T", "half"));
  if (in_t < 0 || qk_t < 0 || qk_t == T_F32 || v_t < 0 || v_t == T_F32) {
    *err = "IN_T must be half|bfloat|float, QK_T and V_T half|bfloat";
    return false;
  }
  LaunchFn f = nullptr;
  if (hd == 128) f = pick_in<128>(in_t, qk_t, v_t, rot != 0, err);
  else if (hd == 64) f = pick_in<64>(in_t, qk_t, v_t, rot != 0, err);
  else *err = "HDIM " + std::to_string(hd) + " not supported (64 or 128)";
  if (!f) return false;
  pl->launch = f;
  pl->threads = 256;
  return true;
}

}  // namespace h3
