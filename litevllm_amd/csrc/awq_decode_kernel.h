// Decode GEMV / skinny GEMM kernel (M <= 32) for the KN layouts (qweight [K, N/8]) on gfx950.
//
// The role of _awq_native_tiled_gemm_heuristic / _split_k at BLOCK_M = 1 .. 32
// (vllm/kernels/triton/awq_fused_gemm.py:1754-1990), built for HBM streaming on MI355X:
//
//  * Work unit = (column tile, k-step): a tile is 16 * WPL packed words (128 * WPL columns),
//    a k-step 32 rows.  Units are numbered tile-major and dealt to the blocks of the grid in
//    equal contiguous ranges ("stream-K"), so every CU streams the same number of bytes
//    whatever the shape.  A block's range touches at most two tiles; the block's NWV waves
//    split each of those tile segments into contiguous k-step shares.
//  * Lane (q = lane / 16, r = lane % 16) owns words tile*16*WPL + r*WPL + w (w < WPL) and,
//    per k-step, rows 8q .. 8q+7.  For each (w, nibble i) the lane builds one 16x32 operand
//    of v_mfma_f32_16x16x32_{f16,bf16} (16 weight columns x 32 k) and multiplies it with the
//    activation operand (32 k x 16 tokens).  Weights are dequantized exactly ((q - z) * s,
//    one rounding) in registers.
//  * Each wave keeps a D-deep ring of k-steps in registers.  Scheduling barriers pin every
//    slot's refill right after the slot is consumed, so D-1 k-steps of loads stay in flight
//    while one is dequantized and multiplied.  Group constants travel with each slot and are
//    prepared when the group changes.
//  * The waves' sums of a tile segment meet in LDS in a fixed tree order.  A tile covered by
//    one block is written directly.  A tile shared by several blocks gets one fp32 partial per
//    block (device-scope stores); after its stores complete, each block bumps the tile's
//    arrival counter, and the last one sums the partials in block (k) order -- fixed, so
//    results are bitwise reproducible for a given shape and plan -- adds the bias once and
//    writes the output.  The reference instead rounds each split to fp16 and atomically adds
//    it (awq_fused_gemm.py:1857-1866) and drops the bias when split (1867-1880).
#pragma once

#include <algorithm>

#include "awq_common.h"
#include "awq_launch.h"

namespace awq {

// Units are dealt in chunks (NWV * D units when that divides the k-steps of a tile, so every
// wave's share of a segment is a whole number of ring turns; 1 otherwise): block b owns
// chunks [b C / B, (b + 1) C / B) of the C chunks.
__host__ __device__ inline int decode_chunk(int ksteps, int nwv, int depth) {
  return (ksteps % (nwv * depth)) == 0 ? nwv * depth : 1;
}
__device__ __forceinline__ int64_t block_begin(int64_t b, int64_t C, int64_t B, int chunk) {
  return (b * C / B) * chunk;
}
// The block that owns unit u.
__device__ __forceinline__ int64_t block_of(int64_t u, int64_t C, int64_t B, int chunk) {
  return ((u / chunk + 1) * B - 1) / C;
}

// LDSW (stream layout only): the weight ring lives in LDS, filled by direct-to-LDS buffer
// loads, so the ring depth costs no registers; activations and group constants ride in a
// register ring of the same depth.
template <int WPL, int MT, int NWV, int D, int SPG, bool SEQ, bool ZP, typename T, bool FAST, bool STREAM,
          int OCC, bool LDSW = false>
__global__ void __launch_bounds__(NWV * 64) __attribute__((amdgpu_waves_per_eu(OCC, OCC)))
decode_kn_kernel(const GemmArgs p, const DecodeWork wk, int scale_bf16) {
  static_assert((SPG & (SPG - 1)) == 0, "");
  static_assert(NWV >= 2 && (NWV & (NWV - 1)) == 0, "power-of-two waves per block");
  static_assert(!LDSW || STREAM, "the LDS weight ring reads the stream layout");
  constexpr int TW = 16 * WPL;        // words per tile
  constexpr int NACC = WPL * 8 * MT;  // f32x4 accumulators per lane
  constexpr int CH = NACC < 16 ? NACC : 16;
  static_assert(NACC % CH == 0, "");
  constexpr int RED_VEC = (NWV / 2) * CH * 64;              // f32x4 of the cross-wave reduction
  constexpr int RING_VEC = LDSW ? NWV * D * 128 * WPL : 0;  // u32x4 of the weight ring
  // the weight ring is dead once the stream ends, so the reduction reuses its space
  __shared__ u32x4 lds_raw[RING_VEC > RED_VEC ? RING_VEC : RED_VEC];
  f32x4* const red = (f32x4*)lds_raw;
  __shared__ int s_last;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform by construction
  const int q = lane >> 4, r = lane & 15;
  const int NW = p.N >> 3;
  const int KS = wk.ksteps;
  const int64_t U = (int64_t)wk.tiles * KS, B = wk.blocks;
  const int chunk = decode_chunk(KS, NWV, D);
  const int64_t C = U / chunk;
  const int64_t b = blockIdx.x;
  const int64_t b0 = block_begin(b, C, B, chunk), b1 = block_begin(b + 1, C, B, chunk);
  if (b0 >= b1) return;  // whole block, uniformly

  // the block's tile segments (the planner keeps b1 - b0 <= KS: at most two)
  const int tA = (int)(b0 / KS);
  const int ksA0 = (int)(b0 - (int64_t)tA * KS);
  const int ksA1 = (int)std::min<int64_t>(KS, b1 - (int64_t)tA * KS);
  const bool two = b1 > (int64_t)(tA + 1) * KS;
  const int ksB1 = two ? (int)(b1 - (int64_t)(tA + 1) * KS) : 0;
  // this wave's contiguous share of each segment
  const int lenA = ksA1 - ksA0, lenB = ksB1;
  const int wA0 = ksA0 + lenA * wave / NWV, nA = ksA0 + lenA * (wave + 1) / NWV - wA0;
  const int wB0 = lenB * wave / NWV, nB = lenB * (wave + 1) / NWV - wB0;
  const int nunits = nA + nB;

  typedef f32x4 Acc[WPL][8][MT];
  Acc acc;   // the segment being computed
  Acc acc0;  // segment A once the wave has moved on to segment B
#pragma unroll
  for (int w = 0; w < WPL; ++w)
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[w][i][mt] = acc0[w][i][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int ngroups = p.K / p.G;
  const uint32_t row_bytes = (uint32_t)NW * 4u;
  if (nunits > 0) {
    const uint32_t w_bytes = STREAM ? (uint32_t)wk.tiles * (uint32_t)KS * 2048u * WPL : (uint32_t)p.K * row_bytes;
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(p.qw, w_bytes);
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(p.a, (uint32_t)((uint64_t)p.M * (uint64_t)p.lda * 2u));
    // the whole activation row offset rides in the VGPR offset, so rows >= M read as zero
    uint32_t x_lane_off[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      x_lane_off[mt] = ((uint32_t)(mt * 16 + r) * (uint32_t)p.lda + 8u * (uint32_t)q) * 2u;
    const __amdgpu_buffer_rsrc_t srs = make_rsrc(p.sc, (uint32_t)((uint64_t)ngroups * p.N * 2u));
    const __amdgpu_buffer_rsrc_t zrs = make_rsrc(p.qz, ZP ? (uint32_t)((uint64_t)ngroups * NW * 4u) : 0u);
    const MagicK mk = magic_consts();

    uint32_t raw[LDSW ? 1 : D][8][WPL];
    u32x4 xr[D][MT];
    WordSZ sz[D][WPL];  // raw constants of each slot's group (used when the group changes)
    ColConst cc[WPL][8];

    // Issue cursor over the wave's units (its share of segment A, then of segment B),
    // advanced one unit per issue.  After the last unit it keeps re-loading that unit with
    // zero activations (their products add exact zeros), so every ring turn is a full one.
    // All per-unit index math is incremental 32-bit scalar arithmetic.
    int it = nA > 0 ? tA : tA + 1;
    int iks = nA > 0 ? wA0 : wB0;
    int ileft = nA > 0 ? nA : nB;  // units left in the current share
    bool in_b = nA == 0, ipast = false;
    auto issue = [&](int slot) {
      const int t = it, ks = iks;  // wave-uniform
      const int word0 = t * TW + r * WPL;
      if constexpr (LDSW) {
        // the unit's run, 1 KiB per instruction, straight into this wave's ring slot: KiB i
        // holds every lane's piece i, lane l's at 16 l
        const int kbase = (int)(((uint32_t)t * (uint32_t)KS + (uint32_t)ks) * 2048u * WPL);
#pragma unroll
        for (int i = 0; i < 2 * WPL; ++i)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              wrs, (__attribute__((address_space(3))) void*)&lds_raw[((wave * D + slot) * 2 * WPL + i) * 64],
              16, (int)((uint32_t)lane * 16u), kbase + 1024 * i, 0, 0);
      } else if constexpr (STREAM) {
        // run of 2 KiB * WPL per unit; lane l's 16-byte piece i at byte 1024 i + 16 l
        const int kbase = (int)(((uint32_t)t * (uint32_t)KS + (uint32_t)ks) * 2048u * WPL);
#pragma unroll
        for (int i = 0; i < 2 * WPL; ++i) {
          const u32x4 v = __builtin_bit_cast(
              u32x4, __builtin_amdgcn_raw_buffer_load_b128(wrs, (int)((uint32_t)lane * 16u), kbase + 1024 * i, 0));
#pragma unroll
          for (int e = 0; e < 4; ++e) raw[slot][(4 * i + e) / WPL][(4 * i + e) % WPL] = v[e];
        }
      } else {
        // rows 8q + j of the lane's WPL words (NW % WPL == 0 keeps the clamped word in bounds)
        const uint32_t lane_off = (uint32_t)(8 * q) * row_bytes + (uint32_t)(word0 < NW ? word0 : 0) * 4u;
        const uint32_t kbase = (uint32_t)ks * 32u * row_bytes;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int soff = (int)(kbase + (uint32_t)j * row_bytes);
          if constexpr (WPL == 4) {
            const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wrs, (int)lane_off, soff, 0));
            raw[slot][j][0] = v[0]; raw[slot][j][1] = v[1]; raw[slot][j][2] = v[2]; raw[slot][j][3] = v[3];
          } else if constexpr (WPL == 2) {
            const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(wrs, (int)lane_off, soff, 0));
            raw[slot][j][0] = v[0]; raw[slot][j][1] = v[1];
          } else {
            raw[slot][j][0] = __builtin_amdgcn_raw_buffer_load_b32(wrs, (int)lane_off, soff, 0);
          }
        }
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        xr[slot][mt] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                     xrs, ipast ? (int)0x80000000 : (int)x_lane_off[mt], ks * 64, 0));
      const int g = ks / SPG;
      const int s_soff = (int)((uint32_t)g * (uint32_t)p.N * 2u);
      const int z_soff = (int)((uint32_t)g * (uint32_t)NW * 4u);
#pragma unroll
      for (int w = 0; w < WPL; ++w) {
        // per-word clamp (columns past N are computed, never stored)
        const uint32_t wc = (uint32_t)min(word0 + w, NW - 1);
        sz[slot][w].s4 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(srs, (int)(16u * wc), s_soff, 0));
        sz[slot][w].zw = ZP ? __builtin_amdgcn_raw_buffer_load_b32(zrs, (int)(4u * wc), z_soff, 0) : 0x88888888u;
      }
      // advance
      if (ileft > 1) {
        --ileft;
        ++iks;
      } else if (!in_b && nB > 0) {
        in_b = true;
        it = tA + 1;
        iks = wB0;
        ileft = nB;
      } else {
        ipast = true;
      }
    };
    auto compute = [&](int slot) {
      const int rs = LDSW ? 0 : slot;
      if constexpr (LDSW) {
        // wait for this slot's direct-to-LDS loads: everything issued for the D - 1 later slots
        // may still be in flight.  The ring is read in inline assembly because the compiler
        // cannot tell the slots apart and would otherwise wait for every load in flight.
        constexpr int kLoadsPerUnit = 2 * WPL + MT + (ZP ? 2 : 1) * WPL;
        constexpr int kAfter = (D - 1) * kLoadsPerUnit;
        static_assert(kAfter <= 63, "vmcnt holds 6 bits");
        __builtin_amdgcn_s_waitcnt((kAfter & 0xF) | ((kAfter >> 4) << 14) | (0x7 << 4) | (0xF << 8));
        // lane l's piece e is at 16 l of KiB e of the slot
        const uint32_t a0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) u32x4*)&lds_raw[(wave * D + slot) * 2 * WPL * 64 + lane];
#pragma unroll
        for (int e = 0; e < 2 * WPL; ++e) {
          u32x4 v;
          asm volatile("ds_read_b128 %0, %1 offset:%2\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(a0), "i"(1024 * e));
#pragma unroll
          for (int c = 0; c < 4; ++c) raw[0][(4 * e + c) / WPL][(4 * e + c) % WPL] = v[c];
        }
      }
#pragma unroll
      for (int w = 0; w < WPL; ++w) {
        uint32_t mlo[4], mhi[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          mlo[v] = pair_lo(raw[rs][2 * v][w], raw[rs][2 * v + 1][w]);
          mhi[v] = pair_hi(raw[rs][2 * v][w], raw[rs][2 * v + 1][w]);
        }
#define AWQ_DECODE_NIB(I)                                                        \
        {                                                                        \
          const u32x4 op = rows_operand<I, FAST, T>(mlo, mhi, cc[w][I], mk);     \
          _Pragma("unroll") for (int mt = 0; mt < MT; ++mt)                      \
              acc[w][I][mt] = MfmaOp<T>::run(op, xr[slot][mt], acc[w][I][mt]);  \
        }
        AWQ_DECODE_NIB(0) AWQ_DECODE_NIB(1) AWQ_DECODE_NIB(2) AWQ_DECODE_NIB(3)
        AWQ_DECODE_NIB(4) AWQ_DECODE_NIB(5) AWQ_DECODE_NIB(6) AWQ_DECODE_NIB(7)
#undef AWQ_DECODE_NIB
      }
    };
    // bookkeeping of the unit being computed: its k-step within its tile and the group
    // whose constants cc holds
    int cks = nA > 0 ? wA0 : wB0;
    int g_cur = -1;
    auto step = [&](int done, int slot) {
      if (done < nunits) {  // wave-uniform bookkeeping of real units
        if (done == nA && nA > 0) {  // moving on to segment B
#pragma unroll
          for (int w = 0; w < WPL; ++w)
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
              for (int mt = 0; mt < MT; ++mt) {
                acc0[w][i][mt] = acc[w][i][mt];
                acc[w][i][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
              }
          cks = wB0;
          g_cur = -1;
        }
        const int g = cks / SPG;
        if (g != g_cur) {
          g_cur = g;
#pragma unroll
          for (int w = 0; w < WPL; ++w) prep_consts<SEQ, FAST>(sz[slot][w], scale_bf16 != 0, cc[w]);
        }
        ++cks;
      }
      compute(slot);
    };

#pragma unroll
    for (int u = 0; u < D; ++u) issue(u);
    __builtin_amdgcn_sched_barrier(0);
    for (int done = 0; done < nunits; done += D) {
#pragma unroll
      for (int u = 0; u < D; ++u) {
        step(done + u, u);
        __builtin_amdgcn_sched_barrier(0);
        issue(u);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // convention for two segments: acc0 = segment A, acc = segment B.  A wave with shares in
    // both moved A to acc0 when B began; one with a share of B only computed it in acc; one
    // with a share of A only moves it now.
    if (two && nA > 0 && nB == 0) {
#pragma unroll
      for (int w = 0; w < WPL; ++w)
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            acc0[w][i][mt] = acc[w][i][mt];
            acc[w][i][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
          }
    }
  }

  // ---- the waves' sums meet in LDS, fixed tree order: ((w0 + w4) + (w2 + w6)) + ... ----
  if constexpr (LDSW) {
    // the reduction reuses the ring's LDS: every wave's last ring reads and direct-to-LDS
    // loads must be over before any wave writes its sums there
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  auto reduce = [&](Acc& A) {
#define AWQ_ACC_AT(IDX) A[(IDX) / (8 * MT)][((IDX) / MT) % 8][(IDX) % MT]
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
  };

  // ---- outputs ----
  // lane (q, r) of wave 0 holds, for accumulator [w][i][mt] element v, token mt*16 + r and
  // column 8 * (t*TW + (4q + v)*WPL + w) + nib_col(i).
  const int M = p.M;
  const int tile_floats = M * TW * 8;  // one partial: [M, TW * 8] fp32
  const __amdgpu_buffer_rsrc_t prs =
      make_rsrc(p.partial, (uint32_t)wk.tiles * (uint32_t)wk.max_contrib * (uint32_t)tile_floats * 4u);
  auto write_out = [&](const Acc& A, int t) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = mt * 16 + r;
      if (m >= M) continue;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
#pragma unroll
        for (int w = 0; w < WPL; ++w) {
          const int word = t * TW + (4 * q + v) * WPL + w;
          if (word >= NW) continue;
          float o[8];
#pragma unroll
          for (int c = 0; c < 8; ++c) o[c] = A[w][col_nib<SEQ>(c)][mt][v];
          if (p.bias) {
#pragma unroll
            for (int c = 0; c < 8; ++c) o[c] += load_bias(p.bias, p.bias_dtype, 8 * word + c);
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
  };
  // partial slot (t, c): [M][TW*8] floats, columns relative to the tile
  auto store_partial = [&](const Acc& A, int t, int c) {
    const uint32_t base = ((uint32_t)t * (uint32_t)wk.max_contrib + (uint32_t)c) * (uint32_t)tile_floats * 4u;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = mt * 16 + r;
      if (m >= M) continue;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
#pragma unroll
        for (int w = 0; w < WPL; ++w) {
          const int lw = (4 * q + v) * WPL + w;  // word within the tile
          const uint32_t off = base + ((uint32_t)m * (uint32_t)(TW * 8) + 8u * (uint32_t)lw) * 4u;
          const f32x4 lo = f32x4{A[w][col_nib<SEQ>(0)][mt][v], A[w][col_nib<SEQ>(1)][mt][v],
                                 A[w][col_nib<SEQ>(2)][mt][v], A[w][col_nib<SEQ>(3)][mt][v]};
          const f32x4 hi = f32x4{A[w][col_nib<SEQ>(4)][mt][v], A[w][col_nib<SEQ>(5)][mt][v],
                                 A[w][col_nib<SEQ>(6)][mt][v], A[w][col_nib<SEQ>(7)][mt][v]};
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, lo), prs, (int)off, 0, kDeviceCoherent);
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, hi), prs, (int)(off + 16u), 0, kDeviceCoherent);
        }
      }
    }
  };
  // the last of the n contributors of tile t sums the partials in contributor (k) order,
  // adds the bias and writes the output (all threads of the block)
  auto reduce_partials = [&](int t, int n) {
    const uint32_t base = (uint32_t)t * (uint32_t)wk.max_contrib * (uint32_t)tile_floats * 4u;
    const uint32_t pstride = (uint32_t)tile_floats * 4u;  // bytes between contributors
    const int ncols = min(TW * 8, p.N - t * TW * 8);
    const int nh = ncols >> 1;  // float2 chunks per row
    for (int idx = tid; idx < M * nh; idx += NWV * 64) {
      const int m = idx / nh, ch = idx - m * nh;
      const uint32_t off = base + ((uint32_t)m * (uint32_t)(TW * 8) + 2u * (uint32_t)ch) * 4u;
      // contributors in groups of 8 whose loads are in flight together; slots past n read
      // as zero (out of the buffer range), and the sum runs in contributor order
      f32x2 sum = {0.f, 0.f};
      for (int c0 = 0; c0 < n; c0 += 8) {
        f32x2 v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t o = (c0 + e < n) ? off + (uint32_t)(c0 + e) * pstride : 0x80000000u;
          v[e] = __builtin_bit_cast(f32x2, __builtin_amdgcn_raw_buffer_load_b64(prs, (int)o, 0, kDeviceCoherent));
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) sum += v[e];
      }
      const int col = t * TW * 8 + 2 * ch;
      if (p.bias) {
        sum[0] += load_bias(p.bias, p.bias_dtype, col);
        sum[1] += load_bias(p.bias, p.bias_dtype, col + 1);
      }
      *(uint32_t*)(p.c + (int64_t)m * p.ldc + col) = pack2<T>(sum[0], sum[1]);
    }
  };
  // one tile segment of the block: write it, or publish its partial and, if last, reduce
  auto finish = [&](Acc& A, int t) {
    reduce(A);
    const int64_t first = block_of((int64_t)t * KS, C, B, chunk);
    const int n = (int)(block_of((int64_t)t * KS + KS - 1, C, B, chunk) - first + 1);
    if (n == 1) {
      if (wave == 0) write_out(A, t);
      return;
    }
    if (wave == 0) {
      store_partial(A, t, (int)(b - first));
      __builtin_amdgcn_s_waitcnt(0);  // the partial stores have completed (device scope)
      if (lane == 0)
        s_last = __hip_atomic_fetch_add(&p.counters[t], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == n - 1;
    }
    __syncthreads();
    const bool last = s_last;
    __syncthreads();  // every wave has read s_last before it can be written again
    if (!last) return;
    reduce_partials(t, n);
    if (tid == 0) __hip_atomic_store(&p.counters[t], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  if (two) {
    finish(acc0, tA);
    finish(acc, tA + 1);
  } else {
    finish(acc, tA);
  }
}

}  // namespace awq

namespace awq_host {
using namespace awq;

template <int WPL, int MT, int NWV, int D, bool SEQ, bool ZP, typename T, bool FAST, bool STREAM, int OCC,
          bool LDSW = false>
inline void launch_t(const GemmArgs& a, const DecodePlan& s, int sbf, hipStream_t st) {
  const DecodeWork wk{s.tiles, s.ksteps, s.blocks, s.max_contrib};
  const int spg = a.G / 32;
  if (spg == 4)
    hipLaunchKernelGGL((decode_kn_kernel<WPL, MT, NWV, D, 4, SEQ, ZP, T, FAST, STREAM, OCC, LDSW>), dim3(s.blocks), dim3(NWV * 64), 0, st, a, wk, sbf);
  else if (spg == 2)
    hipLaunchKernelGGL((decode_kn_kernel<WPL, MT, NWV, D, 2, SEQ, ZP, T, FAST, STREAM, OCC, LDSW>), dim3(s.blocks), dim3(NWV * 64), 0, st, a, wk, sbf);
  else
    hipLaunchKernelGGL((decode_kn_kernel<WPL, MT, NWV, D, 1, SEQ, ZP, T, FAST, STREAM, OCC, LDSW>), dim3(s.blocks), dim3(NWV * 64), 0, st, a, wk, sbf);
}

template <bool SEQ, bool ZP, typename T, bool FAST, bool STREAM>
inline bool launch_sel(const GemmArgs& a, const DecodePlan& s, int sbf, hipStream_t st) {
  if (s.wpl != 1 || s.nwv != 8 || s.depth != 2 || s.occ != 2) return false;
  if (s.mt == 2) launch_t<1, 2, 8, 2, SEQ, ZP, T, FAST, STREAM, 2>(a, s, sbf, st);
  else launch_t<1, 1, 8, 2, SEQ, ZP, T, FAST, STREAM, 2>(a, s, sbf, st);
  return true;
}

}  // namespace awq_host
