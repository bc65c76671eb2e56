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
// K advances in steps of 128 bytes: the A and W slices of a step (2 x 32 KB) are loaded by all 512 threads
// with 16-byte buffer loads (rows past M or N read as zero) one step ahead into registers, then stored into
// the other half of a double-buffered LDS area (one barrier per step). LDS rows are 128 bytes; 16-byte piece p
// of row r is stored at p ^ ((r / 2) % 8), which makes both the staging writes and the operand reads (16 rows
// at one piece per 16-lane pass) bank-conflict free. Workgroups are ordered so that each XCD (own L2) sweeps
// bands of 4 row tiles across the column tiles.
#include "h3hip_internal.h"

#include <algorithm>
#include <cstring>

namespace h3 {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

enum { T_BF16 = 1, T_F16 = 2, T_F32 = 3 };

constexpr int TM = 256, TN = 256, KS = 128;  // tile rows, columns, K bytes per step
constexpr int NWG = 8;                       // waves per workgroup
constexpr int SW = 4;                        // row tiles per band of the tile order
constexpr int STAGE = (TM + TN) * KS;        // LDS bytes per stage

__device__ __forceinline__ int swz(int row, int piece) { return row * KS + ((piece ^ ((row >> 1) & 7)) << 4); }

template <int OT>
__device__ __forceinline__ void store_out(char *p, float v) {
  if constexpr (OT == T_F32) *(float *)p = v;
  else if constexpr (OT == T_BF16) *(__bf16 *)p = (__bf16)v;
  else *(_Float16 *)p = (_Float16)v;
}

template <int OT, int EPI, bool HAS_BIAS>
__global__ __launch_bounds__(NWG * 64) void gemm_q8_kernel(const signed char *__restrict__ A,
                                                           const signed char *__restrict__ W,
                                                           const float *__restrict__ sw, const float *__restrict__ sa,
                                                           char *__restrict__ out, const float *__restrict__ bias,
                                                           const unsigned char *__restrict__ rtype,
                                                           const float *__restrict__ gate, GemmParams p, int ntm,
                                                           int ntn, int ntypes) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int tid = threadIdx.x, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w >> 1, wn = w & 1;

  // tile order: XCD-contiguous ranges (workgroup b runs on XCD b % 8), then bands of SW row tiles
  const int nb = gridDim.x, b = blockIdx.x;
  const int per = nb >> 3, rem = nb & 7, xcd = b & 7, loc = b >> 3;
  const int lid = (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + loc;
  const int band = lid / (SW * ntn), in_band = lid - band * SW * ntn;
  const int rows_in_band = min(SW, ntm - band * SW);
  const int mt = band * SW + in_band % rows_in_band, nt = in_band / rows_in_band;
  const int m0 = mt * TM, n0 = nt * TN;

  // staging: 4 A pieces and 4 W pieces of 16 bytes per thread and step; rows >= M (N) read as zero
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(A + (size_t)m0 * p.a_stride), (short)0, max(0, min(TM, p.M - m0)) * p.a_stride, 0x00020000);
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(W + (size_t)n0 * p.w_stride), (short)0, max(0, min(TN, p.N - n0)) * p.w_stride, 0x00020000);
  i32x4 sa_r[4], sw_r[4];
  auto load = [&](int kt) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int idx = tid + NWG * 64 * i, r = idx >> 3, pc = idx & 7;
      sa_r[i] = __builtin_amdgcn_raw_buffer_load_b128(ra, r * p.a_stride + kt * KS + pc * 16, 0, 0);
      sw_r[i] = __builtin_amdgcn_raw_buffer_load_b128(rw, r * p.w_stride + kt * KS + pc * 16, 0, 0);
    }
  };
  auto store = [&](int buf) {
    char *sA = smem + buf * STAGE, *sW = sA + TM * KS;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int idx = tid + NWG * 64 * i, r = idx >> 3, pc = idx & 7;
      *(i32x4 *)(sA + swz(r, pc)) = sa_r[i];
      *(i32x4 *)(sW + swz(r, pc)) = sw_r[i];
    }
  };

  i32x16 acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0;

  const int nk = p.K / KS;
  load(0);
  store(0);
  __syncthreads();
  for (int kt = 0; kt < nk; kt++) {
    if (kt + 1 < nk) load(kt + 1);
    const char *sA = smem + (kt & 1) * STAGE, *sW = sA + TM * KS;
#pragma unroll
    for (int c = 0; c < KS / 32; c++) {
      i32x4 a[2], bw[4];
#pragma unroll
      for (int i = 0; i < 2; i++) a[i] = *(const i32x4 *)(sA + swz(64 * wm + 32 * i + l32, 2 * c + hl));
#pragma unroll
      for (int j = 0; j < 4; j++) bw[j] = *(const i32x4 *)(sW + swz(128 * wn + 32 * j + l32, 2 * c + hl));
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], bw[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) store((kt + 1) & 1);
    __syncthreads();
  }

  // epilogue: accumulator element e of tile (i, j) is row 64 wm + 32 i + 8 (e / 4) + 4 hl + e % 4, column
  // 128 wn + 32 j + l32
  constexpr int OSZ = OT == T_F32 ? 4 : 2;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int n = n0 + 128 * wn + 32 * j + l32;
    if (n >= p.N) continue;
    const float swn = sw[n];
    const float bn = HAS_BIAS ? bias[n] : 0.0f;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int m = m0 + 64 * wm + 32 * i + 8 * (e >> 2) + 4 * hl + (e & 3);
        if (m >= p.M) continue;
        float v = (float)acc[i][j][e] * sa[m] * swn;
        if constexpr (HAS_BIAS) v += bn;
        if constexpr (EPI == 0) {
          store_out<OT>(out + ((size_t)m * p.c_stride + n) * OSZ, v);
        } else {
          float *x = (float *)out + (size_t)m * p.c_stride + n;
          const int ty = min((int)rtype[m], ntypes - 1);  // types past the gate table's rows clamp to its last
          *x += gate[(size_t)ty * p.g_stride + n] * v;
        }
      }
  }
}

template <int OT, int EPI, bool HAS_BIAS>
int launch_gemm(const Pipeline &pl, hipStream_t stream, const Arg *a, int nargs, const void *params,
                uint32_t params_len, std::string *err) {
  (void)pl;
  if (params_len != sizeof(GemmParams)) {
    *err = "parameter block of " + std::to_string(params_len) + " bytes, expected " +
           std::to_string(sizeof(GemmParams));
    return -1;
  }
  GemmParams p;
  memcpy(&p, params, sizeof p);
  if (p.M < 0 || p.N < 1 || p.K < KS || p.K % KS || p.a_stride < p.K || p.w_stride < p.K || p.c_stride < p.N ||
      p.a_stride % 16 || p.w_stride % 16) {
    *err = "bad shape: M " + std::to_string(p.M) + " N " + std::to_string(p.N) + " K " + std::to_string(p.K) +
           " (a multiple of 128) a_stride " + std::to_string(p.a_stride) + " w_stride " +
           std::to_string(p.w_stride) + " (multiples of 16) c_stride " + std::to_string(p.c_stride);
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
  if (!need(0, (M - 1) * p.a_stride + p.K, "a") || !need(1, (N - 1) * p.w_stride + p.K, "w") ||
      !need(2, N * 4, "sw") || !need(3, M * 4, "sa") || !need(4, ((M - 1) * p.c_stride + N) * OSZ, "out") ||
      (HAS_BIAS && !need(5, N * 4, "bias")))
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
  const int ntm = (p.M + TM - 1) / TM, ntn = (p.N + TN - 1) / TN;
  auto kern = gemm_q8_kernel<OT, EPI, HAS_BIAS>;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, 2 * STAGE);
    if (e != hipSuccess) {
      *err = std::string("hipFuncSetAttribute: ") + hipGetErrorString(e);
      return -1;
    }
    attr_set = true;
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)(ntm * ntn)), dim3(NWG * 64), 2 * STAGE, stream,
                     (const signed char *)a[0].ptr, (const signed char *)a[1].ptr, (const float *)a[2].ptr,
                     (const float *)a[3].ptr, a[4].ptr, HAS_BIAS ? (const float *)a[5].ptr : nullptr,
                     EPI ? (const unsigned char *)a[6].ptr : nullptr, EPI ? (const float *)a[7].ptr : nullptr, p, ntm,
                     ntn, ntypes);
  return 0;
}

template <int OT, int EPI>
LaunchFn pick_bias(bool bias) {
  return bias ? launch_gemm<OT, EPI, true> : launch_gemm<OT, EPI, false>;
}

}  // namespace

// Macros (those of h3metal/ops.py:161-164): WFMT (only 1 = Q8 here), EPI (0 or 1), OUT_T (half | bfloat |
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
  if (wfmt != 1) {
    *err = "weight format " + std::to_string(wfmt) + " not built (only WFMT=1, int8 weights and activations)";
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
  LaunchFn f;
  if (epi) f = pick_bias<T_F32, 1>(hb != 0);
  else if (ot == T_BF16) f = pick_bias<T_BF16, 0>(hb != 0);
  else if (ot == T_F16) f = pick_bias<T_F16, 0>(hb != 0);
  else f = pick_bias<T_F32, 0>(hb != 0);
  pl->launch = f;
  pl->threads = NWG * 64;
  return true;
}

}  // namespace h3
