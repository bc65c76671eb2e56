// Internal declarations shared by the runtime (capi.hip) and the kernel modules.
//
// Parameter blocks keep the reference's byte layout, because the Python launchers
// pack them with struct exactly as the reference does:
//   AttnParams   <- kernels/params.h:41-53, packed by h3metal/ops.py:187-188 ("7if3i")
//   QkRopeParams <- kernels/ops.metal:344-349, packed by h3metal/ops.py:237 ("8ifi")
//   RotQParams   <- kernels/params.h:25-29, packed by h3metal/ops.py:221 ("4i")
//   GemmParams   <- kernels/params.h:7-16, packed by h3metal/ops.py:165-166 ("8i")
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <map>
#include <string>

namespace h3 {

struct AttnParams {
  int Lq;          // query rows
  int L;           // keys (keys >= L are masked)
  int H;           // query heads
  int KVH;         // key/value heads (query head h reads key/value head h / (H / KVH))
  int q_rows;      // rows reserved per head in Q (and in the query scales)
  int k_rows;      // rows reserved per key/value head in K, V (and in the key scales)
  int o_stride;    // elements between rows of the output
  float scale;     // softmax scale times log2(e)
  int causal_off;  // with causal masking: query row i sees keys 0 .. i + causal_off
  int seq_heads;   // heads per sequence: head h writes rows of sequence h / seq_heads
  int seq_rows;    // output rows between consecutive sequences
};
static_assert(sizeof(AttnParams) == 44, "AttnParams must match struct.pack('<7if3i')");

struct QkRopeParams {
  int M, Hq, Hk, Hv, in_stride, out_rows, rot, norm;
  float eps;
  int seq_len;  // rows per sequence: row m is row m % seq_len of sequence m / seq_len
};
static_assert(sizeof(QkRopeParams) == 40, "QkRopeParams must match struct.pack('<8ifi')");

struct RotQParams {
  int M, D;      // rows, features (a multiple of 256)
  int x_stride;  // elements between rows of the input
  int mode;      // 0: input as is; 1: input rows hold [value | gate], the row is value * silu(gate)
};
static_assert(sizeof(RotQParams) == 16, "RotQParams must match struct.pack('<4i')");

struct GemmParams {
  int M;         // rows of A and C (the launcher passes them padded to its tile height)
  int N;         // output features
  int K;         // input features
  int a_stride;  // elements between rows of A
  int c_stride;  // elements between rows of C (or of the residual X)
  int w_stride;  // elements between rows of W
  int groups;    // K / G for group-wise scales (unused by the int8 format)
  int g_stride;  // elements between rows of the gate table
};
static_assert(sizeof(GemmParams) == 32, "GemmParams must match struct.pack('<8i')");

using Macros = std::map<std::string, std::string>;

// One bound buffer argument as the launchers see it: a device address and the
// bytes available from it to the end of its buffer (0 / nullptr when unbound).
struct Arg {
  char *ptr = nullptr;
  uint64_t avail = 0;
};

// Where a launch runs: the stream, and the scratch memory its kernels may use (the attention tail split's
// partial states, the h8 GEMM's widened weights). Launchers never allocate: work that needs more scratch than
// `ws_bytes` either shrinks to fit (the attention split) or fails with a message naming the size it needs.
struct Exec {
  hipStream_t stream = nullptr;
  void *ws = nullptr;
  size_t ws_bytes = 0;
};

// Size of the fixed scratch array that h3_dispatch_static uses instead of the context's workspace.
constexpr size_t STATIC_SCRATCH_BYTES_VALUE = (size_t)32 << 20;

struct Pipeline;
using LaunchFn = int (*)(const Pipeline &pl, const Exec &ex, const Arg *args, int nargs, const void *params,
                         uint32_t params_len, std::string *err);

// A selected kernel specialisation (what h3_pipeline returns).
struct Pipeline {
  std::string name;   // "module:fn(macros)" for messages
  LaunchFn launch = nullptr;
  int threads = 0;    // threads per workgroup of the launch
  int ival[8] = {};   // module-specific specialisation values
};

// Module factories: fill `pl` for (fn, macros) or return false with a message.
bool make_attention(const std::string &fn, const Macros &m, Pipeline *pl, std::string *err);
bool make_ops(const std::string &fn, const Macros &m, Pipeline *pl, std::string *err);
bool make_rot_q8(const Macros &m, Pipeline *pl, std::string *err);  // module "ops", function "rot_q8"
bool make_gemm(const std::string &fn, const Macros &m, Pipeline *pl, std::string *err);

// Wave64 lane exchanges inside a 32-lane half wave, shared by the row kernels: the value of lane (lane ^ S).
// DPP for S = 1, 2 (quad_perm) and 8 (row_ror:8, a 16-lane rotation by 8), ds_swizzle's xor mode (no LDS
// memory access) for S = 4, 16.
template <int S>
__device__ __forceinline__ float xshfl(float v) {
  const int x = __builtin_bit_cast(int, v);
  if constexpr (S == 1) return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, true));
  else if constexpr (S == 2) return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, true));
  else if constexpr (S == 8) return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, true));
  else return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(x, 0x1F | (S << 10)));
}

// v[i] += c * (v[i] of the lane selected by the DPP control CTRL), for all N values (N even), as assembly: the
// compiler keeps a separate DPP move for the builtin form. A DPP read needs two wait states after a VALU write of
// its source; each assembly statement starts with its own s_nop 1 before its (at most eight) reads, so nothing the
// compiler schedules can come between the wait and the reads, and the statement writes only its own values.
#define H3_DPP_FMAC_STAGE(CTRL)                                                                                   \
  do {                                                                                                            \
    static_assert(N % 2 == 0, "an even number of values per lane");                                             \
    _Pragma("unroll") for (int i = 0; i + 8 <= N; i += 8) asm volatile(                                          \
        "s_nop 1\n\tv_fmac_f32_dpp %0, %0, %8 " CTRL "\n\tv_fmac_f32_dpp %1, %1, %8 " CTRL                       \
        "\n\tv_fmac_f32_dpp %2, %2, %8 " CTRL "\n\tv_fmac_f32_dpp %3, %3, %8 " CTRL                                \
        "\n\tv_fmac_f32_dpp %4, %4, %8 " CTRL "\n\tv_fmac_f32_dpp %5, %5, %8 " CTRL                                \
        "\n\tv_fmac_f32_dpp %6, %6, %8 " CTRL "\n\tv_fmac_f32_dpp %7, %7, %8 " CTRL                                \
        : "+v"(v[i]), "+v"(v[i + 1]), "+v"(v[i + 2]), "+v"(v[i + 3]), "+v"(v[i + 4]), "+v"(v[i + 5]),           \
          "+v"(v[i + 6]), "+v"(v[i + 7])                                                                         \
        : "v"(c));                                                                                                \
    if constexpr (N % 8 >= 4) asm volatile(                                                                       \
        "s_nop 1\n\tv_fmac_f32_dpp %0, %0, %4 " CTRL "\n\tv_fmac_f32_dpp %1, %1, %4 " CTRL                       \
        "\n\tv_fmac_f32_dpp %2, %2, %4 " CTRL "\n\tv_fmac_f32_dpp %3, %3, %4 " CTRL                                \
        : "+v"(v[N / 8 * 8]), "+v"(v[N / 8 * 8 + 1]), "+v"(v[N / 8 * 8 + 2]), "+v"(v[N / 8 * 8 + 3])             \
        : "v"(c));                                                                                                \
    if constexpr (N % 4 == 2)                                                                                     \
      asm volatile("s_nop 1\n\tv_fmac_f32_dpp %0, %0, %2 " CTRL "\n\tv_fmac_f32_dpp %1, %1, %2 " CTRL             \
                   : "+v"(v[N - 2]), "+v"(v[N - 1])                                                              \
                   : "v"(c));                                                                                     \
  } while (0)

// One cross-lane stage of a Walsh-Hadamard transform over lane bit LS, on N values per lane: every lane
// computes own + c * partner with c = +1 on the lower lane of a pair and -1 on the upper one. The lower lane gets
// a + b, the upper b - a = -(a - b); partners share every other lane bit, so after stages over a set of lane bits
// a lane holds its true values times (-1)^(number of those bits set in the lane id), which the caller folds into
// its final scale (an exact sign change). The product with c is exact and the one rounding is that of the sum,
// the same as for a + b or a - b (rounding is sign-symmetric). For LS = 1, 2, 8 the shuffled value is the
// multiplicand of an fmac that reads it straight through DPP (H3_DPP_FMAC_STAGE).
template <int LS, int N>
__device__ __forceinline__ void hadamard_lane_stage(float (&v)[N], float c) {
  if constexpr (LS == 1) {
    H3_DPP_FMAC_STAGE("quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf bound_ctrl:1");
  } else if constexpr (LS == 2) {
    H3_DPP_FMAC_STAGE("quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf bound_ctrl:1");
  } else if constexpr (LS == 8) {
    H3_DPP_FMAC_STAGE("row_ror:8 row_mask:0xf bank_mask:0xf bound_ctrl:1");
  } else {
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = __builtin_fmaf(xshfl<LS>(v[i]), c, v[i]);
  }
}

// LDS-direct buffer loads: lane i's 16 (dma16) or 4 (dma4) bytes land at LDS byte m0 + 16 i (+ 4 i); offsets
// beyond the descriptor's range read as zero. Written as assembly so that the compiler does not make every LDS
// read wait for them; the caller waits itself (vmcnt) before the barrier that publishes the data. M0 must be
// wave-uniform; the s_nop gives the load the wait state it needs after the M0 write.
__device__ __forceinline__ void dma16(unsigned m0, unsigned voff, __amdgpu_buffer_rsrc_t r) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(m0), "v"(voff), "s"(r)
               : "memory", "m0");
}
__device__ __forceinline__ void dma4(unsigned m0, unsigned voff, __amdgpu_buffer_rsrc_t r) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds" ::"s"(m0), "v"(voff), "s"(r)
               : "memory", "m0");
}

// Compute units of the current device (0 if unknown).
int cu_count();
// Scratch bytes the attention launcher's tail split can use at most on a device with `cus` compute units
// (what h3_open reserves, so that ordinary dispatches never wait for memory).
size_t attention_workspace_max(int cus);

// Helpers for macro parsing in the factories.
bool macro_int(const Macros &m, const char *key, int def, int *out, std::string *err);
std::string macro_str(const Macros &m, const char *key, const char *def);

}  // namespace h3
