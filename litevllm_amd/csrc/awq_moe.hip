// Mixture-of-experts: routing (softmax -> top-k -> renormalise), expert-stack stream packing,
// route lists, the combine, planning, and the f16 instantiations of the grouped GEMM kernels
// (awq_moe_kernel.h); bf16 ones live in awq_moe_misc.hip.
#include "awq_moe_kernel.h"

namespace awq {

__device__ __forceinline__ float load_logit(const void* p, int dtype, int64_t i) {
  if (dtype == AWQ_DTYPE_F16) return h_bits2f(((const uint16_t*)p)[i]);
  if (dtype == AWQ_DTYPE_BF16) return bf_bits2f(((const uint16_t*)p)[i]);
  return ((const float*)p)[i];
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Whole-wave max / sum through DPP (row reductions by quad permutes and mirrors, then the row
// broadcasts to lane 63), read back as a wave-uniform value: a few cycles per step where the
// LDS crossbar shuffles above take about a hundred.
__device__ __forceinline__ int dpp_i(int v, int ctrl, int row_mask) {
  switch (ctrl) {  // the control word must be a constant
    case 0xB1: return __builtin_amdgcn_update_dpp(v, v, 0xB1, 0xF, 0xF, false);
    case 0x4E: return __builtin_amdgcn_update_dpp(v, v, 0x4E, 0xF, 0xF, false);
    case 0x141: return __builtin_amdgcn_update_dpp(v, v, 0x141, 0xF, 0xF, false);
    case 0x140: return __builtin_amdgcn_update_dpp(v, v, 0x140, 0xF, 0xF, false);
    case 0x142: return __builtin_amdgcn_update_dpp(v, v, 0x142, 0xA, 0xF, false);
    default: return __builtin_amdgcn_update_dpp(v, v, 0x143, 0xC, 0xF, false);
  }
}
template <bool MAX>
__device__ __forceinline__ float dpp_reduce(float v) {
  auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
  // quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror: every lane holds
  // its row's result
  v = op(v, __int_as_float(dpp_i(__float_as_int(v), 0xB1, 0xF)));
  v = op(v, __int_as_float(dpp_i(__float_as_int(v), 0x4E, 0xF)));
  v = op(v, __int_as_float(dpp_i(__float_as_int(v), 0x141, 0xF)));
  v = op(v, __int_as_float(dpp_i(__float_as_int(v), 0x140, 0xF)));
  // row_bcast:15 into rows 1 and 3, row_bcast:31 into rows 2 and 3 (other lanes add their
  // own value back for the sum: only lane 63 is read)
  const float b15 = __int_as_float(dpp_i(__float_as_int(v), 0x142, 0xA));
  v = (MAX || ((__lane_id() >> 4) & 1)) ? op(v, b15) : v;
  const float b31 = __int_as_float(dpp_i(__float_as_int(v), 0x143, 0xC));
  v = (MAX || (__lane_id() >> 5)) ? op(v, b31) : v;
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// x (> 0, finite) rounded once to fp16 (dt F16) or bf16 (dt BF16), returned as fp32: the double
// is first rounded to fp32 toward zero with the inexact bit kept in the last place (round to
// odd), which leaves the second rounding to nearest-even the correctly rounded result (fp32
// carries more than two bits beyond either 16-bit format, subnormal fp16 included).
__device__ __forceinline__ float round_prob(double x, int dt) {
  float f = (float)x;
  if ((double)f != x) {
    uint32_t b = __float_as_uint(f);
    if ((double)f > x) b -= 1;  // positive: the nearest fp32 at or below x
    f = __uint_as_float(b | 1u);
  }
  return dt == AWQ_DTYPE_F16 ? h_bits2f(f2h_bits(f)) : bf_bits2f(f2bf_bits(f));
}
__device__ __forceinline__ float round_to(float x, int dt) {
  if (dt == AWQ_DTYPE_F16) return h_bits2f(f2h_bits(x));
  if (dt == AWQ_DTYPE_BF16) return bf_bits2f(f2bf_bits(x));
  return x;
}

// Routing of one token per wave (E <= 256), two dtype flows:
//  * fp32 (the Gemma4 router, models/gemma4/moe.py:106-116): p = softmax(fp32(logits)) in fp32;
//    the top_k largest p (ties: lower expert id first) in descending order; with renormalize,
//    w = p / sum (or / max(sum, 1e-8) with AWQ_ROUTE_CLAMP_SUM), the sum taken in slot order;
//  * AWQ_ROUTE_SOFTMAX_IN_LOGITS_DTYPE (fused_moe.py:12-15, 16-bit logits): p = softmax(logits)
//    rounded once to the logits dtype (exp and sum in fp64, so p is the correctly rounded
//    quotient), top-k on those values, and w = dt(fp32(p) / fp32(dt(sum of the selected p))),
//    torch's arithmetic for 16-bit tensors (fp32 math, one rounding per operation).
// out_w receives w in w_dtype (F32, F16 or BF16; RNE from fp32).
__global__ void __launch_bounds__(256) moe_route_kernel(const void* logits, int64_t ld, int dtype, int64_t T,
                                                        int E, int topk, uint32_t flags, void* out_w, int w_dtype,
                                                        int32_t* out_ids) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;  // whole wave
  const bool in_dt = (flags & AWQ_ROUTE_SOFTMAX_IN_LOGITS_DTYPE) && dtype != AWQ_DTYPE_F32;
  if (!in_dt && E <= 64) {
    // fp32 flow, one probability per lane: DPP max and sum, then top_k rounds of (max, lowest
    // lane holding it) -- the choices and order of the rank pass below
    const float x = lane < E ? load_logit(logits, dtype, t * ld + lane) : -INFINITY;
    const float mx = dpp_reduce<true>(x);
    const float ex = lane < E ? expf(x - mx) : 0.f;
    const float sum = dpp_reduce<false>(ex);
    float cur = lane < E ? ex / sum : -1.f;  // -1: not selectable
    float mine = 0.f, sel_sum = 0.f;
    int mine_id = 0;
    for (int k = 0; k < topk; ++k) {
      const float bv = dpp_reduce<true>(cur);
      const uint64_t m = __ballot(cur == bv);
      const int src = __ffsll((unsigned long long)m) - 1;
      if (lane == k) {
        mine = bv;
        mine_id = src;
      }
      sel_sum += bv;
      if (lane == src) cur = -1.f;
    }
    if (lane < topk) {
      float w = mine;
      if (flags & AWQ_ROUTE_RENORMALIZE) w = mine / ((flags & AWQ_ROUTE_CLAMP_SUM) ? fmaxf(sel_sum, 1e-8f) : sel_sum);
      const int64_t o = t * topk + lane;
      if (w_dtype == AWQ_DTYPE_F32) ((float*)out_w)[o] = w;
      else ((uint16_t*)out_w)[o] = w_dtype == AWQ_DTYPE_F16 ? f2h_bits(w) : f2bf_bits(w);
      out_ids[o] = mine_id;
    }
    return;
  }
  float v[4];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = lane + 64 * j;
    v[j] = e < E ? load_logit(logits, dtype, t * ld + e) : -INFINITY;
    mx = fmaxf(mx, v[j]);
  }
  mx = wave_max(mx);
  if (in_dt) {
    double ev[4], sd = 0.0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = lane + 64 * j;
      ev[j] = e < E ? exp((double)v[j] - (double)mx) : 0.0;  // v - mx exact in fp64
      sd += ev[j];
    }
    sd = wave_sum_f64(sd);
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = (lane + 64 * j) < E ? round_prob(ev[j] / sd, dtype) : -1.f;
  } else {
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = lane + 64 * j;
      v[j] = e < E ? expf(v[j] - mx) : 0.f;
      s += v[j];
    }
    s = wave_sum(s);
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = (lane + 64 * j) < E ? v[j] / s : -1.f;  // -1: not selectable
  }
  float mine = 0.f, sel_sum = 0.f;
  int mine_id = 0;
  if (E <= 64) {
    // one probability per lane: its rank among the E (larger first, equal ones by lower id)
    // in one pass over the lanes, then slot k is the lane of rank k -- the same choices, in
    // the same order, as the repeated arg-max below
    const int vb = __float_as_int(v[0]);
    const float vi = v[0];
    int rank = 0;
    for (int j = 0; j < E; ++j) {  // wave-uniform
      const float vj = __int_as_float(__builtin_amdgcn_readlane(vb, j));
      rank += (vj > vi || (vj == vi && j < lane)) ? 1 : 0;
    }
    for (int k = 0; k < topk; ++k) {
      const uint64_t m = __ballot(lane < E && rank == k);
      const int src = m ? __ffsll((unsigned long long)m) - 1 : 0;
      const float bv = __int_as_float(__builtin_amdgcn_readlane(vb, src));
      if (lane == k) {
        mine = bv;
        mine_id = src;
      }
      sel_sum += bv;
    }
  } else for (int k = 0; k < topk; ++k) {
    float bv = -1.f;
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (v[j] > bv) { bv = v[j]; bi = lane + 64 * j; }  // j ascending: lower id wins ties
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const float ov = __shfl_xor(bv, o);
      const int oi = __shfl_xor(bi, o);
      if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (lane + 64 * j == bi) v[j] = -1.f;
    if (lane == k) { mine = bv; mine_id = bi; }
    sel_sum += bv;
  }
  if (lane < topk) {
    float w = mine;
    if (flags & AWQ_ROUTE_RENORMALIZE) {
      if (in_dt) {
        w = round_to(mine / round_to(sel_sum, dtype), dtype);
      } else {
        w = mine / ((flags & AWQ_ROUTE_CLAMP_SUM) ? fmaxf(sel_sum, 1e-8f) : sel_sum);
      }
    }
    const int64_t o = t * topk + lane;
    if (w_dtype == AWQ_DTYPE_F32) ((float*)out_w)[o] = w;
    else ((uint16_t*)out_w)[o] = w_dtype == AWQ_DTYPE_F16 ? f2h_bits(w) : f2bf_bits(w);
    out_ids[o] = mine_id;
  }
}

// Expert stack [E][K][NW] (AutoAWQ words) -> [E][tiles][K/32] runs of 2048 bytes: the decode
// stream layout (pack_stream_kernel), tile words chosen by moe_word.  Lane l = 16q + r holds
// rows 32s + 8q + 2v, 2v + 1 (v = 0..3) of word moe_word(t, r) paired into their low 16-bit
// halves (u32 v of piece 0, byte 16 l + 4 v of the run) and their high halves (piece 1, byte
// 1024 + 16 l + 4 v), so the kernels form the MFMA operands without byte permutes (T = 512
// gate_up 64.8 -> 64.1 us against unpaired rows).
__global__ void __launch_bounds__(256) moe_pack_stream_kernel(const uint32_t* __restrict__ in,
                                                              uint32_t* __restrict__ out, int64_t K,
                                                              int64_t NW, int64_t tiles, int half,
                                                              int64_t E) {
  const int64_t KS = K / 32;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= E * tiles * KS * 64) return;
  const int l = (int)(idx & 63);
  const int64_t run = idx >> 6;  // (e * tiles + t) * KS + s
  const int64_t s = run % KS;
  const int64_t et = run / KS;
  const int64_t t = et % tiles, e = et / tiles;
  const int q = l >> 4, r = l & 15;
  const int w = moe_word((int)t, r, half, (int)NW);
  const uint32_t* src = in + e * K * NW;
  uint32_t* dst = out + run * 512;
  uint32_t rows[8];
  for (int j = 0; j < 8; ++j) rows[j] = w >= 0 ? src[(s * 32 + 8 * q + j) * NW + w] : 0u;
  for (int v = 0; v < 4; ++v) {
    dst[l * 4 + v] = pair_lo(rows[2 * v], rows[2 * v + 1]);        // piece 0
    dst[256 + l * 4 + v] = pair_hi(rows[2 * v], rows[2 * v + 1]);  // piece 1
  }
}

// Route lists: block e collects the routes r (in increasing order) whose id is e, 1024 ids per
// round.  The ids of the first kAlignPre rounds are all requested before the first round runs
// (one memory wait instead of one per round); later rounds load their own.
constexpr int kAlignPre = 4, kAlignThreads = 1024;
__global__ void __launch_bounds__(kAlignThreads) moe_align_kernel(const void* ids, int id64, int R, int* lists,
                                                                  int* counts) {
  constexpr int NWV = kAlignThreads / 64;
  __shared__ int s_wcnt[NWV];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int e = blockIdx.x;
  int* list = lists + (int64_t)e * R;
  auto load_id = [&](int idx) -> int {
    if (idx >= R) return -1;
    return id64 ? (int)((const int64_t*)ids)[idx] : ((const int32_t*)ids)[idx];
  };
  int count = 0;
  auto round = [&](int base, int id) {
    const int idx = base + tid;
    const bool hit = id == e;
    const uint64_t m = __ballot(hit);
    if (lane == 0) s_wcnt[wave] = __popcll(m);
    __syncthreads();
    int off = count, tot = count;
#pragma unroll
    for (int w = 0; w < NWV; ++w) {
      off += w < wave ? s_wcnt[w] : 0;
      tot += s_wcnt[w];
    }
    if (hit) list[off + __popcll(m & ((1ull << lane) - 1ull))] = idx;
    __syncthreads();  // s_wcnt is read by every wave before the next round writes it
    count = tot;
  };
  int pre[kAlignPre];
#pragma unroll
  for (int u = 0; u < kAlignPre; ++u) pre[u] = load_id(u * kAlignThreads + tid);
#pragma unroll
  for (int u = 0; u < kAlignPre; ++u)
    if (u * kAlignThreads < R) round(u * kAlignThreads, pre[u]);  // block-uniform
  for (int base = kAlignPre * kAlignThreads; base < R; base += kAlignThreads) round(base, load_id(base + tid));
  if (tid == 0) counts[e] = count;
}

// out[t, 4c .. 4c+3] = round(sum over j of y[t * topk + j, 4c ..]) in j order; routes whose
// expert id is outside [0, E) contribute nothing.
template <typename T>
__global__ void __launch_bounds__(256) moe_combine_kernel(const float* __restrict__ y, const void* ids, int id64,
                                                          int E, int64_t T_tok, int64_t H, int topk,
                                                          uint16_t* __restrict__ out, int64_t ldo) {
  // T_tok * H / 4 < 2^31 (the caller's 32-bit offset limits): 32-bit index arithmetic
  const uint32_t idx = blockIdx.x * 256u + threadIdx.x;
  const uint32_t hq = (uint32_t)(H >> 2);
  if ((int64_t)idx >= T_tok * (int64_t)hq) return;
  const int64_t t = idx / hq, c = idx - (uint32_t)t * hq;
  f32x4 s = {0.f, 0.f, 0.f, 0.f};
  int j = 0;
  // eight routes at a time: their ids and rows are all requested before any is added (the
  // rows of every route exist, so the loads need not wait for the id checks); the sum still
  // runs in j order
  for (; j + 8 <= topk; j += 8) {
    int id[8];
    f32x4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t rt = t * topk + j + u;
      id[u] = id64 ? (int)((const int64_t*)ids)[rt] : ((const int32_t*)ids)[rt];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = *(const f32x4*)(y + (t * topk + j + u) * H + 4 * c);
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (id[u] >= 0 && id[u] < E) s += v[u];
  }
  for (; j < topk; ++j) {
    const int64_t rt = t * topk + j;
    const int id = id64 ? (int)((const int64_t*)ids)[rt] : ((const int32_t*)ids)[rt];
    if (id < 0 || id >= E) continue;
    s += *(const f32x4*)(y + rt * H + 4 * c);
  }
  u32x2 st;
  st[0] = pack2<T>(s[0], s[1]);
  st[1] = pack2<T>(s[2], s[3]);
  *(u32x2*)(out + t * ldo + 4 * c) = st;
}

}  // namespace awq

namespace awq_host {
using namespace awq;

static int launch_status() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? AWQ_OK : AWQ_ERR_LAUNCH;
}

int64_t moe_tiles(int64_t N, int gate_up) {
  return gate_up ? cdiv(N / 16, 8) : cdiv(N / 8, 16);
}

int64_t moe_stream_bytes(int64_t E, int64_t K, int64_t N, int gate_up) {
  return E * moe_tiles(N, gate_up) * (K / 32) * 2048;
}

int launch_moe_pack_stream(const int32_t* in, int32_t* out, int64_t E, int64_t K, int64_t N, int gate_up,
                           hipStream_t st) {
  const int64_t tiles = moe_tiles(N, gate_up);
  const int64_t n = E * tiles * (K / 32) * 64;
  if (n == 0) return AWQ_OK;
  hipLaunchKernelGGL(moe_pack_stream_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, st, (const uint32_t*)in,
                     (uint32_t*)out, K, N / 8, tiles, gate_up ? (int)(N / 16) : 0, E);
  return launch_status();
}

int launch_moe_route(const void* logits, int64_t ld, int dtype, int64_t T, int E, int topk, uint32_t flags,
                     void* out_w, int w_dtype, int32_t* out_ids, hipStream_t st) {
  if (T == 0) return AWQ_OK;
  hipLaunchKernelGGL(moe_route_kernel, dim3((unsigned)cdiv(T, 4)), dim3(256), 0, st, logits, ld, dtype, T, E, topk,
                     flags, out_w, w_dtype, out_ids);
  return launch_status();
}

template <int MODE>
static void launch_gemm_f16(const MoeArgs& a, int E, int mt, bool zp, hipStream_t st) {
  if (mt == 2) zp ? launch_moe_gemm_t<MODE, 2, true, f16, false>(a, E, st) : launch_moe_gemm_t<MODE, 2, false, f16, false>(a, E, st);
  else zp ? launch_moe_gemm_t<MODE, 1, true, f16, false>(a, E, st) : launch_moe_gemm_t<MODE, 1, false, f16, false>(a, E, st);
}

// expected routes per expert from which the grouped MFMA kernels take over
constexpr int kMoeMfmaMinRoutes = 16;

// 16-token tiles per wave group, from the expected routes per expert
// (two tiles at most: the per-group and the scaled sums of four tiles would not fit the
// registers of two waves per SIMD; larger route counts take more passes over the row loop)
static int moe_mt(int64_t R, int E) {
  const int64_t avg = R / (E > 0 ? E : 1);
  return avg <= 12 ? 1 : 2;
}

MoeWorkspace moe_workspace(int64_t T, int64_t H, int64_t I, int E, int topk, int act_bytes) {
  MoeWorkspace w{};
  const int64_t R = T * topk;
  auto al = [](int64_t x) { return (x + 255) & ~(int64_t)255; };
  w.counts = 0;
  w.lists = al(w.counts + (int64_t)E * 4);
  w.tmp = al(w.lists + (int64_t)E * R * 4);
  w.y = al(w.tmp + R * I * act_bytes);
  w.total = al(w.y + R * H * 4);
  return w;
}

int launch_moe(const MoeCall& c, hipStream_t st) {
  const int64_t R = c.T * c.topk;
  const int act_bytes = 2;
  const MoeWorkspace w = moe_workspace(c.T, c.H, c.I, c.E, c.topk, act_bytes);
  char* ws = (char*)c.workspace;
  int* counts = (int*)(ws + w.counts);
  int* lists = (int*)(ws + w.lists);
  uint16_t* tmp = (uint16_t*)(ws + w.tmp);
  float* y = (float*)(ws + w.y);
  const bool zp = c.gu_qz != nullptr;
  const int mt = moe_mt(R, c.E);
  const int sbf = c.scale_dtype == AWQ_DTYPE_BF16 ? 1 : 0;
  const bool mfma = R >= (int64_t)kMoeMfmaMinRoutes * c.E && (c.H % 64) == 0 && (c.I % 64) == 0 && (c.G & (c.G - 1)) == 0;
  // few routes: the stream kernels collect each expert's routes from the ids themselves
  const bool scan = !mfma && R <= kMoeScanMaxR;

  if (!scan) {
    hipLaunchKernelGGL(moe_align_kernel, dim3((unsigned)c.E), dim3(kAlignThreads), 0, st, c.ids, c.id64, (int)R, lists,
                       counts);
    if (launch_status() != AWQ_OK) return AWQ_ERR_LAUNCH;
  }

  MoeArgs gu{};
  gu.a = (const uint16_t*)c.x;
  gu.qw = (const uint32_t*)c.gu_qw;
  gu.sc = (const uint16_t*)c.gu_sc;
  gu.qz = (const uint32_t*)c.gu_qz;
  gu.lists = scan ? nullptr : lists;
  gu.counts = scan ? nullptr : counts;
  gu.ids = c.ids;
  gu.id64 = c.id64;
  gu.rw = c.rw;
  gu.out = tmp;
  gu.lda = c.ldx;
  gu.ldo = c.I;
  gu.R = (int)R;
  gu.topk = c.topk;
  gu.K = (int)c.H;
  gu.N = (int)(2 * c.I);
  gu.G = c.G;
  gu.half = (int)(c.I / 8);
  gu.tiles = (int)moe_tiles(2 * c.I, 1);
  gu.rows_a = (int)c.T;
  gu.rw_dtype = c.rw_dtype;
  gu.act_kind = c.act_kind;

  MoeArgs dn = gu;
  dn.a = tmp;
  dn.qw = (const uint32_t*)c.dn_qw;
  dn.sc = (const uint16_t*)c.dn_sc;
  dn.qz = (const uint32_t*)c.dn_qz;
  dn.out = y;
  dn.lda = c.I;
  dn.ldo = c.H;
  dn.K = (int)c.I;
  dn.N = (int)c.H;
  dn.half = 0;
  dn.tiles = (int)moe_tiles(c.H, 0);
  dn.rows_a = (int)R;

  if (mfma) {
    // many routes per expert: each dequantized weight operand feeds up to six 16-route tiles
    launch_moe_mfma(gu, dn, c.E, zp, c.act_dtype, sbf, st);
  } else if (c.act_dtype == AWQ_DTYPE_F16 && !sbf) {
    launch_gemm_f16<0>(gu, c.E, mt, zp, st);
    if (launch_status() != AWQ_OK) return AWQ_ERR_LAUNCH;
    launch_gemm_f16<1>(dn, c.E, mt, zp, st);
  } else {
    if (!launch_moe_misc(gu, dn, c.E, zp, c.act_dtype, sbf, st)) return AWQ_ERR_UNSUPPORTED;
  }
  if (launch_status() != AWQ_OK) return AWQ_ERR_LAUNCH;

  const int64_t n = c.T * (c.H / 4);
  if (c.act_dtype == AWQ_DTYPE_BF16)
    hipLaunchKernelGGL(moe_combine_kernel<bf16>, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, st, y, c.ids, c.id64, c.E,
                       c.T, c.H, c.topk, (uint16_t*)c.out, c.ldo);
  else
    hipLaunchKernelGGL(moe_combine_kernel<f16>, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, st, y, c.ids, c.id64, c.E,
                       c.T, c.H, c.topk, (uint16_t*)c.out, c.ldo);
  return launch_status();
}

}  // namespace awq_host
