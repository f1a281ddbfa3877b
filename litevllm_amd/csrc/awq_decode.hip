// Decode GEMV / skinny GEMM (M <= 32) for the KN layouts (qweight [K, N/8]) on gfx950.
//
// The role of _awq_native_tiled_gemm_heuristic / _split_k at BLOCK_M = 1 .. 32
// (vllm/kernels/triton/awq_fused_gemm.py:1754-1990), built for HBM streaming on MI355X:
//
//  * Block = NWV waves on one column tile of 16 * WPL packed words (128 * WPL columns).
//    Lane (q = lane / 16, r = lane % 16) owns words tile*16*WPL + r*WPL + w (w < WPL) and,
//    per 32-row k-step, rows 8q .. 8q+7.  For each (w, nibble i) the lane builds one 16x32
//    operand of v_mfma_f32_16x16x32_{f16,bf16} (16 weight columns x 32 k) and multiplies it
//    with the activation operand (32 k x 16 tokens).
//  * Work is cut in whole quantization groups: split s of the grid covers groups
//    [s*I, (s+1)*I); the NWV waves of a block take contiguous, balanced shares of those.
//  * Each wave keeps a D-deep ring of k-steps in registers.  Scheduling barriers pin every
//    slot's refill right after the slot is consumed, so D-1 k-steps of loads stay in flight
//    while one is dequantized and multiplied (the compiler would otherwise sink the refills
//    to the end of the loop body and drain the ring every turn).
//  * Partial sums of the waves meet in LDS in a fixed tree order.  With nsplit > 1 every
//    block publishes its fp32 partial tile with device-scope stores, waits for them, and
//    bumps the tile's arrival counter; the block that arrives last sums all partials in
//    split order (fixed, so results are bitwise reproducible), adds the bias once and writes
//    the output.  The reference instead rounds each split to fp16 and atomically adds it
//    (awq_fused_gemm.py:1857-1866) and drops the bias when split (1867-1880).
#include <algorithm>

#include "awq_common.h"
#include "awq_launch.h"

namespace awq {

template <int WPL, int MT, int NWV, int D, int SPG, bool SEQ, bool ZP, typename T, bool FAST, bool STREAM>
__global__ void __launch_bounds__(NWV * 64) decode_kn_kernel(const GemmArgs p, int scale_bf16) {
  static_assert(!STREAM || WPL == 4, "the decode stream layout holds 4 words per lane");
  constexpr int NACC = WPL * 8 * MT;  // f32x4 accumulators per lane
  constexpr int CH = NACC < 16 ? NACC : 16;
  constexpr int IG = D / SPG;         // groups per ring turn
  static_assert(D % SPG == 0, "ring depth must hold whole groups");
  static_assert(NWV >= 2 && (NWV & (NWV - 1)) == 0, "power-of-two waves per block");
  static_assert(NACC % CH == 0, "");
  __shared__ f32x4 red[(NWV / 2) * CH * 64];
  __shared__ int s_last;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR) by construction
  const int q = lane >> 4, r = lane & 15;
  const int NW = p.N >> 3;
  const int tile = blockIdx.x, split = blockIdx.y;
  const int word0 = tile * 16 * WPL + r * WPL;
  // per-word clamp for the group constants (columns past N are computed, never stored)
  int wsz[WPL];
#pragma unroll
  for (int w = 0; w < WPL; ++w) wsz[w] = min(word0 + w, NW - 1);

  // groups of this wave
  const int ngroups = p.K / p.G;
  const int gs0 = split * p.groups_per_split;
  const int gs1 = min(ngroups, gs0 + p.groups_per_split);
  const int ng = max(0, gs1 - gs0);
  const int gbase = ng / NWV, gextra = ng - gbase * NWV;
  const int wg0 = gs0 + wave * gbase + min(wave, gextra);
  const int wg1 = wg0 + gbase + (wave < gextra ? 1 : 0);

  f32x4 acc[WPL][8][MT];
#pragma unroll
  for (int w = 0; w < WPL; ++w)
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[w][i][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (wg0 < wg1) {
    const int ks_begin = wg0 * SPG, ks_end = wg1 * SPG;  // k-steps [ks_begin, ks_end)
    const int ks_last = ks_end - 1;
    // KN layouts: lane (q, r) reads rows 8q + j of its WPL words (NW % WPL == 0 keeps the
    // clamped word in bounds).  Stream layout: each (tile, k-step) is 8 contiguous 1 KiB
    // chunks, chunk j holding, for lane l, the 16 bytes this mapping needs from row 8q + j.
    const int KS = p.K / 32;
    const uint32_t row_bytes = (uint32_t)NW * 4u;
    const uint32_t w_bytes = STREAM ? (uint32_t)cdiv_u(NW, 64) * (uint32_t)p.K * 256u : (uint32_t)p.K * row_bytes;
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(p.qw, w_bytes);
    const uint32_t lane_off = STREAM ? (uint32_t)lane * 16u
                                     : (uint32_t)(8 * q) * row_bytes + (uint32_t)(word0 < NW ? word0 : 0) * 4u;
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(p.a, (uint32_t)((uint64_t)p.M * (uint64_t)p.lda * 2u));
    // the whole row offset rides in the VGPR offset, so rows >= M read as zero
    uint32_t x_lane_off[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      x_lane_off[mt] = ((uint32_t)(mt * 16 + r) * (uint32_t)p.lda + 8u * (uint32_t)q) * 2u;
    const __amdgpu_buffer_rsrc_t srs = make_rsrc(p.sc, (uint32_t)((uint64_t)ngroups * p.N * 2u));
    const __amdgpu_buffer_rsrc_t zrs = make_rsrc(p.qz, ZP ? (uint32_t)((uint64_t)ngroups * NW * 4u) : 0u);
    const MagicK mk = magic_consts();

    uint32_t raw[D][8][WPL];
    u32x4 xr[D][MT];
    WordSZ szc[IG][WPL];  // raw constants of the groups of the ring turn being computed
    ColConst cc[WPL][8];

    auto issue = [&](int ks, uint32_t (&dst)[8][WPL], u32x4 (&xd)[MT]) {
      // wave-uniform base of the k-step
      const uint32_t kbase = STREAM ? ((uint32_t)tile * (uint32_t)KS + (uint32_t)ks) * 8192u
                                    : (uint32_t)ks * 32u * row_bytes;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int soff = (int)(kbase + (uint32_t)j * (STREAM ? 1024u : row_bytes));
        if constexpr (WPL == 4) {
          const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wrs, (int)lane_off, soff, 0));
          dst[j][0] = v[0]; dst[j][1] = v[1]; dst[j][2] = v[2]; dst[j][3] = v[3];
        } else if constexpr (WPL == 2) {
          const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(wrs, (int)lane_off, soff, 0));
          dst[j][0] = v[0]; dst[j][1] = v[1];
        } else {
          dst[j][0] = __builtin_amdgcn_raw_buffer_load_b32(wrs, (int)lane_off, soff, 0);
        }
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        xd[mt] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, (int)x_lane_off[mt], ks * 64, 0));
    };
    auto issue_sz = [&](int g, WordSZ (&dst)[WPL]) {
      const int s_soff = (int)((uint32_t)g * (uint32_t)p.N * 2u);
      const int z_soff = (int)((uint32_t)g * (uint32_t)NW * 4u);
#pragma unroll
      for (int w = 0; w < WPL; ++w) {
        dst[w].s4 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(srs, (int)(16u * (uint32_t)wsz[w]), s_soff, 0));
        dst[w].zw = ZP ? __builtin_amdgcn_raw_buffer_load_b32(zrs, (int)(4u * (uint32_t)wsz[w]), z_soff, 0) : 0x88888888u;
      }
    };
    auto compute = [&](const uint32_t (&rw)[8][WPL], const u32x4 (&xv)[MT]) {
#pragma unroll
      for (int w = 0; w < WPL; ++w) {
        uint32_t mlo[4], mhi[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          mlo[u] = pair_lo(rw[2 * u][w], rw[2 * u + 1][w]);
          mhi[u] = pair_hi(rw[2 * u][w], rw[2 * u + 1][w]);
        }
#define AWQ_DECODE_NIB(I)                                                        \
        {                                                                        \
          const u32x4 op = rows_operand<I, FAST, T>(mlo, mhi, cc[w][I], mk);     \
          _Pragma("unroll") for (int mt = 0; mt < MT; ++mt)                      \
              acc[w][I][mt] = MfmaOp<T>::run(op, xv[mt], acc[w][I][mt]);         \
        }
        AWQ_DECODE_NIB(0) AWQ_DECODE_NIB(1) AWQ_DECODE_NIB(2) AWQ_DECODE_NIB(3)
        AWQ_DECODE_NIB(4) AWQ_DECODE_NIB(5) AWQ_DECODE_NIB(6) AWQ_DECODE_NIB(7)
#undef AWQ_DECODE_NIB
      }
    };
    auto prep = [&](const WordSZ (&szv)[WPL]) {
#pragma unroll
      for (int w = 0; w < WPL; ++w) prep_consts<SEQ, FAST>(szv[w], scale_bf16 != 0, cc[w]);
    };

    // prologue: the first D k-steps.  Slots past the wave's range re-load its last k-step
    // (cache hits, never used).  The slot that starts a group also carries that group's
    // raw constants, so they travel (and are waited for) with its weight words.
#pragma unroll
    for (int u = 0; u < D; ++u) {
      const int ks = min(ks_begin + u, ks_last);
      if (u % SPG == 0) issue_sz(ks / SPG, szc[u / SPG]);
      issue(ks, raw[u], xr[u]);
    }
    __builtin_amdgcn_sched_barrier(0);

    int ks0 = ks_begin;
    for (; ks0 + D <= ks_end; ks0 += D) {
#pragma unroll
      for (int u = 0; u < D; ++u) {
        if (u % SPG == 0) prep(szc[u / SPG]);
        compute(raw[u], xr[u]);
        __builtin_amdgcn_sched_barrier(0);
        const int nks = min(ks0 + u + D, ks_last);
        if (u % SPG == 0) issue_sz(nks / SPG, szc[u / SPG]);
        issue(nks, raw[u], xr[u]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // tail (only when the wave's range is not a multiple of D k-steps)
#pragma unroll
    for (int u = 0; u < D; ++u) {
      if (ks0 + u < ks_end) {
        if (u % SPG == 0) prep(szc[u / SPG]);
        compute(raw[u], xr[u]);
      }
    }
  }

  // ---- cross-wave reduction, fixed tree order: ((w0 + w4) + (w2 + w6)) + ... ----
#define AWQ_ACC_AT(IDX) acc[(IDX) / (8 * MT)][((IDX) / MT) % 8][(IDX) % MT]
#pragma unroll
  for (int c0 = 0; c0 < NACC; c0 += CH) {
#pragma unroll
    for (int half = NWV / 2; half >= 1; half >>= 1) {
      if (wave >= half && wave < 2 * half) {
#pragma unroll
        for (int c = 0; c < CH; ++c) red[((wave - half) * CH + c) * 64 + lane] = AWQ_ACC_AT(c0 + c);
      }
      __syncthreads();
      if (wave < half) {
#pragma unroll
        for (int c = 0; c < CH; ++c) AWQ_ACC_AT(c0 + c) += red[(wave * CH + c) * 64 + lane];
      }
      __syncthreads();
    }
  }
#undef AWQ_ACC_AT

  // lane (q, r) of wave 0 holds, for accumulator [w][i][mt] element v, token mt*16 + r and
  // column 8 * (tile*16*WPL + (4q + v)*WPL + w) + nib_col(i).
  const int M = p.M, N = p.N;
  if (p.nsplit == 1) {
    if (wave == 0) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = mt * 16 + r;
        if (m >= M) continue;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
#pragma unroll
          for (int w = 0; w < WPL; ++w) {
            const int word = tile * 16 * WPL + (4 * q + v) * WPL + w;
            if (word >= NW) continue;
            float o[8];
#pragma unroll
            for (int cidx = 0; cidx < 8; ++cidx) o[cidx] = acc[w][col_nib<SEQ>(cidx)][mt][v];
            if (p.bias) {
#pragma unroll
              for (int cidx = 0; cidx < 8; ++cidx) o[cidx] += load_bias(p.bias, p.bias_dtype, 8 * word + cidx);
            }
            u32x4 st;
            st[0] = pack2<T>(o[0], o[1]);
            st[1] = pack2<T>(o[2], o[3]);
            st[2] = pack2<T>(o[4], o[5]);
            st[3] = pack2<T>(o[6], o[7]);
            *(u32x4*)(p.c + (int64_t)m * p.ldc + 8 * word) = st;
          }
        }
      }
    }
    return;
  }

  // ---- split-K: publish the fp32 partial tile, the last block of the tile reduces ----
  const uint32_t part_bytes = (uint32_t)p.nsplit * (uint32_t)M * (uint32_t)N * 4u;
  const __amdgpu_buffer_rsrc_t prs = make_rsrc(p.partial, part_bytes);
  if (wave == 0) {
    const uint32_t split_off = (uint32_t)split * (uint32_t)M * (uint32_t)N * 4u;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = mt * 16 + r;
      if (m >= M) continue;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
#pragma unroll
        for (int w = 0; w < WPL; ++w) {
          const int word = tile * 16 * WPL + (4 * q + v) * WPL + w;
          if (word >= NW) continue;
          const uint32_t off = ((uint32_t)m * (uint32_t)N + 8u * (uint32_t)word) * 4u;
          const f32x4 lo = f32x4{acc[w][col_nib<SEQ>(0)][mt][v], acc[w][col_nib<SEQ>(1)][mt][v],
                                 acc[w][col_nib<SEQ>(2)][mt][v], acc[w][col_nib<SEQ>(3)][mt][v]};
          const f32x4 hi = f32x4{acc[w][col_nib<SEQ>(4)][mt][v], acc[w][col_nib<SEQ>(5)][mt][v],
                                 acc[w][col_nib<SEQ>(6)][mt][v], acc[w][col_nib<SEQ>(7)][mt][v]};
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, lo), prs, (int)(off + split_off), 0, kDeviceCoherent);
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, hi), prs, (int)(off + split_off + 16u), 0, kDeviceCoherent);
        }
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // the partial stores have completed (device scope)
  __syncthreads();
  if (tid == 0) {
    const int prev = __hip_atomic_fetch_add(&p.counters[tile], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == p.nsplit - 1);
  }
  __syncthreads();
  if (!s_last) return;
  const int col0 = tile * 16 * WPL * 8;
  const int ncols = min(16 * WPL * 8, N - col0);
  const int nq = ncols >> 2;  // float4 chunks per row
  const uint32_t sstride = (uint32_t)M * (uint32_t)N * 4u;
  for (int idx = tid; idx < M * nq; idx += NWV * 64) {
    const int m = idx / nq, cq = idx - m * nq;
    const int col = col0 + 4 * cq;
    const uint32_t off = ((uint32_t)m * (uint32_t)N + (uint32_t)col) * 4u;
    f32x4 sum = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(prs, (int)off, 0, kDeviceCoherent));
    for (int sp = 1; sp < p.nsplit; ++sp)
      sum += __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(prs, (int)(off + (uint32_t)sp * sstride), 0, kDeviceCoherent));
    if (p.bias) {
#pragma unroll
      for (int e = 0; e < 4; ++e) sum[e] += load_bias(p.bias, p.bias_dtype, col + e);
    }
    u32x2 st;
    st[0] = pack2<T>(sum[0], sum[1]);
    st[1] = pack2<T>(sum[2], sum[3]);
    *(u32x2*)(p.c + (int64_t)m * p.ldc + col) = st;
  }
  if (tid == 0) __hip_atomic_store(&p.counters[tile], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace awq

namespace awq_host {
using namespace awq;

// ---- planning ----
// Candidate (words per lane, ring depth, waves) shapes and split counts are scored by how
// evenly one round of resident blocks covers the chip, with at least kMinGroupsPerWave
// groups of k-steps per wave where the problem allows.
DecodePlan plan_decode(int64_t M, int64_t N, int64_t K, int64_t G, int split_k, DecodeMode mode) {
  DecodePlan s{};
  s.mt = (M > 16) ? 2 : 1;
  s.nwv = 4;
  const int64_t nw = N / 8;
  const int64_t ng = K / G;
  const int64_t cus = num_cus();
  int wpl;
  if (mode == kDecodeStream) {
    wpl = 4;
  } else if (mode == kDecodeWide) {
    // widest tile that still gives >= 1 tile per CU, else the widest that divides N
    wpl = 4;
    while (wpl > 1 && (nw % wpl) != 0) wpl >>= 1;
    while (wpl > 1 && cdiv(nw, 16 * wpl) < cus) wpl >>= 1;
    if (s.mt == 2 && wpl > 2) wpl = 2;
  } else {
    wpl = 1;
  }
  s.wpl = wpl;
  s.depth = wpl == 4 ? 4 : 8;  // 8 k-steps of 4-word rows would not fit the register file
  s.tiles = (int)cdiv(nw, 16 * wpl);
  int64_t ns;
  if (split_k > 0) {
    ns = split_k;
  } else {
    // one block per CU (4 waves of up to 512 VGPRs): splits so that tiles x splits covers
    // the CUs evenly, each wave keeping >= 1 group
    const int64_t max_ns = std::max<int64_t>(1, ng / s.nwv);
    int64_t best = 1;
    double best_score = -1e30;
    for (int64_t c = 1; c <= max_ns; ++c) {
      const int64_t blocks = (int64_t)s.tiles * c;
      const double rounds = (double)cdiv(blocks, cus);
      const double fill = (double)blocks / (rounds * (double)cus);
      const double score = fill - 0.01 * (double)c - 0.3 * (rounds - 1.0);
      if (score > best_score + 1e-9) {
        best_score = score;
        best = c;
      }
    }
    ns = best;
  }
  ns = std::max<int64_t>(1, std::min<int64_t>(ns, ng));
  s.groups_per_split = (int)cdiv(ng, ns);
  s.nsplit = (int)cdiv(ng, s.groups_per_split);  // no empty partitions
  s.ws_bytes = 0;
  if (s.nsplit > 1) s.ws_bytes = kCounterBytes + (size_t)s.nsplit * (size_t)M * (size_t)N * sizeof(float);
  return s;
}

template <int WPL, int MT, int NWV, int D, bool SEQ, bool ZP, typename T, bool FAST, bool STREAM = false>
static void launch_t(const GemmArgs& a, const DecodePlan& s, int sbf, hipStream_t st) {
  dim3 grid(s.tiles, s.nsplit);
  const int spg = a.G / 32;
  if (spg == 4)
    hipLaunchKernelGGL((decode_kn_kernel<WPL, MT, NWV, D, 4, SEQ, ZP, T, FAST, STREAM>), grid, dim3(NWV * 64), 0, st, a, sbf);
  else if (spg == 2)
    hipLaunchKernelGGL((decode_kn_kernel<WPL, MT, NWV, D, 2, SEQ, ZP, T, FAST, STREAM>), grid, dim3(NWV * 64), 0, st, a, sbf);
  else
    hipLaunchKernelGGL((decode_kn_kernel<WPL, MT, NWV, D, 1, SEQ, ZP, T, FAST, STREAM>), grid, dim3(NWV * 64), 0, st, a, sbf);
}

// Stream layout (AutoAWQ nibble order, fp16 activations and scales): 4 words per lane.
template <bool ZP>
static bool launch_stream(const GemmArgs& a, const DecodePlan& s, hipStream_t st) {
  if (s.wpl != 4 || s.nwv != 4 || s.depth != 4) return false;
  if (s.mt == 2) launch_t<4, 2, 4, 4, false, ZP, f16, true, true>(a, s, 0, st);
  else launch_t<4, 1, 4, 4, false, ZP, f16, true, true>(a, s, 0, st);
  return true;
}

// Main path (AutoAWQ interleave, fp16 activations and scales): every tile width.
template <bool ZP>
static bool launch_main(const GemmArgs& a, const DecodePlan& s, hipStream_t st) {
#define AWQ_CASE(W, MTV, NV, DD)                                                                   \
  if (s.wpl == W && s.mt == MTV && s.nwv == NV && s.depth == DD) {                                 \
    launch_t<W, MTV, NV, DD, false, ZP, f16, true>(a, s, 0, st);                                   \
    return true;                                                                                   \
  }
  AWQ_CASE(1, 1, 4, 8) AWQ_CASE(2, 1, 4, 8) AWQ_CASE(4, 1, 4, 4)
  AWQ_CASE(1, 2, 4, 8) AWQ_CASE(2, 2, 4, 8)
#ifdef AWQ_DECODE_TUNE_SET
  AWQ_DECODE_TUNE_SET
#endif
#undef AWQ_CASE
  return false;
}

// Other dtype / layout combinations: one word per lane (plans made with wide = false).
template <bool SEQ, bool ZP, typename T, bool FAST>
static bool launch_other(const GemmArgs& a, const DecodePlan& s, int sbf, hipStream_t st) {
  if (s.mt == 2) launch_t<1, 2, 4, 8, SEQ, ZP, T, FAST>(a, s, sbf, st);
  else launch_t<1, 1, 4, 8, SEQ, ZP, T, FAST>(a, s, sbf, st);
  return true;
}

bool launch_decode(const GemmArgs& a, const DecodePlan& s, DecodeMode mode, bool seq, bool zp,
                   int act, int sdt, hipStream_t st) {
  const int sbf = (sdt == AWQ_DTYPE_BF16) ? 1 : 0;
  if (mode == kDecodeStream) {
    if (seq || act != AWQ_DTYPE_F16 || sdt != AWQ_DTYPE_F16) return false;
    return zp ? launch_stream<true>(a, s, st) : launch_stream<false>(a, s, st);
  }
  if (mode == kDecodeWide) return zp ? launch_main<true>(a, s, st) : launch_main<false>(a, s, st);
  if (s.wpl != 1) return false;
  if (act == AWQ_DTYPE_F16) {
    if (sdt == AWQ_DTYPE_F16) {  // seq layout, fast dequant
      return zp ? launch_other<true, true, f16, true>(a, s, 0, st) : launch_other<true, false, f16, true>(a, s, 0, st);
    }
    if (seq) return zp ? launch_other<true, true, f16, false>(a, s, sbf, st) : launch_other<true, false, f16, false>(a, s, sbf, st);
    return zp ? launch_other<false, true, f16, false>(a, s, sbf, st) : launch_other<false, false, f16, false>(a, s, sbf, st);
  }
  if (seq) return zp ? launch_other<true, true, bf16, false>(a, s, sbf, st) : launch_other<true, false, bf16, false>(a, s, sbf, st);
  return zp ? launch_other<false, true, bf16, false>(a, s, sbf, st) : launch_other<false, false, bf16, false>(a, s, sbf, st);
}

}  // namespace awq_host
