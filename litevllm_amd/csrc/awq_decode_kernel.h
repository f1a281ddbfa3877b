// Decode GEMV / skinny GEMM kernel (M <= 32) for the KN layouts (qweight [K, N/8]) and the
// decode stream copy on gfx950.
//
// The role of _awq_native_tiled_gemm_heuristic / _split_k at BLOCK_M = 1 .. 32
// (vllm/kernels/triton/awq_fused_gemm.py:1754-1990), built for HBM streaming on MI355X:
//
//  * Work unit = (column tile, k-step): a tile is 16 packed words (128 columns), a k-step 32
//    rows.  Each tile's k-steps are cut into `splits` ranges (the reference's split-K rule),
//    one per block, and the block's waves take contiguous shares of its range, so a block
//    never leaves its tile.
//  * Lane (q = lane / 16, r = lane % 16) owns word tile*16 + r and, per k-step, rows
//    8q .. 8q+7.  For each nibble i the lane builds one 32 k x 16 column operand of
//    v_mfma_f32_16x16x32_{f16,bf16} and multiplies the activations (16 tokens x 32 k) by it,
//    so lane (q, r) accumulates tokens 4q .. 4q+3 of column 8 * word + nib_col(i).
//  * The weights enter the MFMA as the exact biased integers B + q (biased_operand: one
//    AND-OR per pair of rows, no subtraction), and one more MFMA per k-step against ones sums
//    the activations; when a group ends, (B + z) times that sum is taken off each column's sum
//    and the result is multiplied once by the group's fp32 scale.  So the weights are
//    (q - z) * s, never rounded -- the reference's M = 1 formulation, b = (q - z) * s kept in
//    fp32 (awq_fused_gemm.py:1966-1971); its tl.dot path for M > 1 rounds b to fp16 first
//    (1973-1976), which this kernel does not.
//  * Each wave keeps a D-deep ring of k-steps in registers.  Scheduling barriers pin every
//    slot's refill right after the slot is consumed, so D-1 k-steps of loads stay in flight
//    while one is dequantized and multiplied.
//  * The waves' sums meet in LDS in a fixed tree order.  With one split the block writes the
//    tile; otherwise each block stores an fp32 partial (device-scope stores), bumps the tile's
//    arrival counter once its stores are complete, and the last block sums the partials in
//    split (k) order -- fixed, so results are bitwise reproducible for a given shape and
//    split count -- adds the bias once and writes the output.  The reference instead rounds
//    each split to fp16 and atomically adds it (awq_fused_gemm.py:1857-1866) and drops the
//    bias when split (1867-1880).
#pragma once

#include <algorithm>

#include "awq_common.h"
#include "awq_launch.h"

namespace awq {

// MT: 16-token MFMA tiles (M <= 16 MT).  ONE: M == 1, so only element 0 of lane q = 0's
// accumulators holds a real token and only that element is scaled and reduced.
// SBF: scales are bf16 (fp16 otherwise).  STREAM: weights in the decode stream layout.
// XL (ONE, stream layout): the block's slice of the activation row is staged in LDS once by
// DMA and every lane reads its k-slice from there (the MFMA's other 15 rows repeat row 0 and
// are never read back), instead of a 16-byte load per lane and k-step.
template <int MT, int NWV, int D, int SPG, bool SEQ, bool ZP, typename T, bool SBF, bool STREAM, bool ONE,
          int OCC, bool XL>
__global__ void __launch_bounds__(NWV * 64) __attribute__((amdgpu_waves_per_eu(OCC, OCC)))
decode_kn_kernel(const GemmArgs p_in, const DecodeWork wk) {
  static_assert((SPG & (SPG - 1)) == 0, "");
  static_assert(!XL || (ONE && STREAM), "");
  static_assert(NWV >= 2 && (NWV & (NWV - 1)) == 0, "power-of-two waves per block");
  static_assert(!ONE || MT == 1, "");
  // Biased operands (one AND-OR or permute per pair of rows, the zero taken off per group) pay
  // when a group spans several k-steps of one token tile, and always for bf16 (whose exact
  // integer operands need conversions); otherwise the exact integers q - z (one more packed
  // subtraction per pair of rows, a single multiply-add per group) are cheaper.
  constexpr bool BIASED = (SPG >= 2 && MT == 1) || (!std::is_same<T, f16>::value && !(MT == 2 && SPG == 1));
  constexpr int MROWS = ONE ? 1 : 16 * MT;  // token rows a wave can hold
  // row y of a row-exact launch: row y's M = 1 problem (the call itself otherwise)
  const BlockXY bxy = decode_block(p_in.rows, wk.tiles * wk.splits);
  const GemmArgs p = row_slice(p_in, wk.tiles, wk.tiles * wk.splits * p_in.M * 128, bxy.y);
  __shared__ float red[NWV * MROWS * 128];  // every wave's sums: [wave][token][tile column]
  __shared__ int s_last;
  extern __shared__ __align__(16) unsigned char xsm[];  // XL: activations k0 * 32 .. k1 * 32 of row 0

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform by construction
  const int q = lane >> 4, r = lane & 15;
  const int NW = p.N >> 3;
  const int KS = wk.ksteps, S = wk.splits;
  const int t = bxy.x / S, part = bxy.x - t * S;
  // the block's k-step range of tile t, then this wave's contiguous share of it
  const int k0 = min(part * wk.per, KS), k1 = min(k0 + wk.per, KS);
  const int len = k1 - k0;
  const int w0 = k0 + len * wave / NWV;
  const int nunits = k0 + len * (wave + 1) / NWV - w0;
  const int word = t * 16 + r;  // the lane's packed word

  f32x4 acc[8][MT];  // the current group's sums, biased integer weights B + q
  f32x4 ax[MT];      // the current group's activation sums (the bias correction)
  f32x4 tot[8][MT];  // the scaled sums of the groups done (general case)
  float tot1[8];     // the same when ONE (element 0 only)
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    tot1[i] = 0.f;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[i][mt] = tot[i][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) ax[mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int ngroups = p.K / p.G;
  const uint32_t row_bytes = (uint32_t)NW * 4u;
  if constexpr (XL) {
    // 16-byte pieces i of the block's activation slice; wave w issues DMA instructions
    // w, w + NWV, ... of 64 pieces
    const u32x4 xrs4 = rsrc_words(p.a, (uint32_t)((uint64_t)p.lda * 2u));
    const uint32_t xsm_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)xsm;
    const int npieces = len * 4;
    for (int j = wave; j * 64 < npieces; j += NWV) {
      const int i = j * 64 + lane;
      lds_dma16(xrs4, xsm_base + (uint32_t)j * 1024u, i < npieces ? (uint32_t)(k0 * 64 + i * 16) : 0x80000000u, 0u);
    }
  }
  if (nunits > 0) {
    const uint32_t w_bytes = STREAM ? (uint32_t)wk.tiles * (uint32_t)KS * 2048u : (uint32_t)p.K * row_bytes;
    const uint32_t x_bytes = (uint32_t)((uint64_t)p.M * (uint64_t)p.lda * 2u);
    const uint32_t s_bytes = (uint32_t)((uint64_t)ngroups * p.N * 2u);
    const uint32_t z_bytes = ZP ? (uint32_t)((uint64_t)ngroups * NW * 4u) : 0u;
    // the whole activation row offset rides in the VGPR offset, so rows >= M read as zero
    uint32_t x_lane_off[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      x_lane_off[mt] = ((uint32_t)(mt * 16 + r) * (uint32_t)p.lda + 8u * (uint32_t)q) * 2u;
    const BiasK bk = bias_consts<T>();
    const MagicK mk = magic_consts();
    const u32x4 ones = {ones2<T>(), ones2<T>(), ones2<T>(), ones2<T>()};
    // per-column clamp (columns past N are computed, never stored)
    const uint32_t wc = (uint32_t)min(word, NW - 1);
    const uint32_t w_lane_off = STREAM ? (uint32_t)lane * 16u : (uint32_t)(8 * q) * row_bytes + wc * 4u;

    uint32_t raw[D][8];
    u32x4 xr[D][MT];
    WordSZ sz[D];    // raw constants of each slot's group (used when the group changes)
    uint32_t zwc;    // zero word of the current group (biased operands)
    uint32_t zm[8];  // biased zeros of the current group (exact integer operands)
    u32x4 s4;        // scales of the current group (the word's 8 columns, raw 16-bit values)

    // Issue cursor over the wave's units, advanced one unit per issue.  Past the last unit the
    // ring's refills go through empty buffer descriptors (zeros, no memory traffic), so every
    // ring turn is a whole one; all per-unit index math is 32-bit scalar arithmetic.
    // A unit's scales and zeros are loaded only where a group starts (or in the first turn,
    // which includes the wave's first unit): prep reads no other slot's.
    int iks = w0, ileft = nunits;
    // Stream layout: weight piece 0 of the next unit (its low-half rows) into slot `slot`, without
    // advancing the cursor; a unit's compute issues it as soon as those rows are used up (after
    // nibble 3) and the refill after the compute skips it (skip_w0), so half of each refill goes
    // out half a unit earlier (N = 24576: M = 2 .. 16 0.4 - 0.8% faster, M = 1 0 - 0.2%; bitwise
    // equal; A/Bs on two boxes)
    auto issue_w0 = [&](int slot) {
      const bool past = ileft <= 0;
      const __amdgpu_buffer_rsrc_t wrs = make_rsrc(p.qw, past ? 0u : w_bytes);
      const int kbase = (int)(((uint32_t)t * (uint32_t)KS + (uint32_t)iks) * 2048u);
      const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wrs, (int)w_lane_off, kbase, kStreamNT));
#pragma unroll
      for (int c = 0; c < 4; ++c) raw[slot][c] = v[c];
    };
    auto issue = [&](int slot, bool first_turn, bool skip_w0 = false) {
      const int ks = iks;  // wave-uniform
      const bool past = ileft <= 0;
      ++iks;
      --ileft;
      const __amdgpu_buffer_rsrc_t wrs = make_rsrc(p.qw, past ? 0u : w_bytes);
      const __amdgpu_buffer_rsrc_t xrs = make_rsrc(p.a, past ? 0u : x_bytes);
      const __amdgpu_buffer_rsrc_t srs = make_rsrc(p.sc, past ? 0u : s_bytes);
      const __amdgpu_buffer_rsrc_t zrs = make_rsrc(p.qz, past ? 0u : z_bytes);
      if constexpr (STREAM) {
        // the unit's 2 KiB run; lane l's 16-byte piece e at byte 1024 e + 16 l
        const int kbase = (int)(((uint32_t)t * (uint32_t)KS + (uint32_t)ks) * 2048u);
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          if (e == 0 && skip_w0) continue;
          const u32x4 v = __builtin_bit_cast(
              u32x4, __builtin_amdgcn_raw_buffer_load_b128(wrs, (int)w_lane_off, kbase + 1024 * e, kStreamNT));
#pragma unroll
          for (int c = 0; c < 4; ++c) raw[slot][4 * e + c] = v[c];
        }
      } else {
        // rows 8q + j of the lane's word
        const uint32_t kbase = (uint32_t)ks * 32u * row_bytes;
#pragma unroll
        for (int j = 0; j < 8; ++j)
          raw[slot][j] = __builtin_amdgcn_raw_buffer_load_b32(wrs, (int)w_lane_off, (int)(kbase + (uint32_t)j * row_bytes), 0);
      }
      if constexpr (!XL)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          xr[slot][mt] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, (int)x_lane_off[mt], ks * 64, 0));
      // (the 16-wave M == 1 kernel without LDS activations keeps the per-unit loads: holding
      // a slot's constants across turns would not fit its 128 registers)
      // The constants are read once, like the weights, and take the same non-temporal policy:
      // with the default policy the M = 1, N = 24576 launch measured 0.2 us longer (11.04 against
      // 10.83 us, bitwise equal results).
      if (first_turn || (ks & (SPG - 1)) == 0 || (ONE && !XL)) {  // wave-uniform
        const int g = ks / SPG;
        sz[slot].s4 = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(srs, (int)(16u * wc), (int)((uint32_t)g * (uint32_t)p.N * 2u), kStreamNT));
        sz[slot].zw = ZP ? __builtin_amdgcn_raw_buffer_load_b32(zrs, (int)(4u * wc), (int)((uint32_t)g * (uint32_t)NW * 4u), kStreamNT)
                         : 0x88888888u;
      }
    };
    int cks_x = w0;  // the next unit to compute (XL reads its activations from LDS)
    auto xop = [&](int slot, int mt) -> u32x4 {
      if constexpr (XL) return *(const u32x4*)(xsm + ((cks_x - k0) * 32 + 8 * q) * 2);
      else return xr[slot][mt];
    };
    // FRESH: the group's first unit (its MFMAs start from zero); early_w0: refill piece 0 of the
    // slot once its rows are used up (stream layout)
    auto compute = [&](int slot, auto fresh, bool early_w0 = false) {
      constexpr bool FRESH = decltype(fresh)::value;
      uint32_t mlo[4], mhi[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        if constexpr (STREAM) {  // rows arrive paired (pack_stream_kernel)
          mlo[v] = raw[slot][v];
          mhi[v] = raw[slot][4 + v];
        } else {
          mlo[v] = pair_lo(raw[slot][2 * v], raw[slot][2 * v + 1]);
          mhi[v] = pair_hi(raw[slot][2 * v], raw[slot][2 * v + 1]);
        }
      }
      u32x4 xv[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) xv[mt] = xop(slot, mt);
      ++cks_x;
#define AWQ_DECODE_NIB(I)                                                                      \
      {                                                                                        \
        const u32x4 op = BIASED ? biased_operand<I, T>(mlo, mhi, bk) : int_operand<I, T>(mlo, mhi, zm[I], mk); \
        _Pragma("unroll") for (int mt = 0; mt < MT; ++mt)                                      \
            acc[I][mt] = MfmaOp<T>::run(xv[mt], op, FRESH ? f32x4{0.f, 0.f, 0.f, 0.f} : acc[I][mt]); \
      }
      AWQ_DECODE_NIB(0) AWQ_DECODE_NIB(1) AWQ_DECODE_NIB(2) AWQ_DECODE_NIB(3)
      if constexpr (STREAM) {
        if (early_w0) {  // wave-uniform
          __builtin_amdgcn_sched_barrier(0);
          issue_w0(slot);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      AWQ_DECODE_NIB(4) AWQ_DECODE_NIB(5) AWQ_DECODE_NIB(6) AWQ_DECODE_NIB(7)
#undef AWQ_DECODE_NIB
      if constexpr (BIASED)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          ax[mt] = MfmaOp<T>::run(xv[mt], ones, FRESH ? f32x4{0.f, 0.f, 0.f, 0.f} : ax[mt]);
    };
    // tot += the scaled sums s * sum x (q - z) of the group just finished, from the biased
    // sums and the activation sums (ZERO: the sums restart from zero)
    auto flush = [&](auto zero) {
      if constexpr (!BIASED) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const int c = nib_col<SEQ>(i);
            const uint16_t sb = (uint16_t)(s4[c >> 1] >> (16 * (c & 1)));
            const float sf = SBF ? bf_bits2f(sb) : h_bits2f(sb);
            if constexpr (ONE) tot1[i] += acc[i][mt][0] * sf;
            else tot[i][mt] += acc[i][mt] * sf;
            if constexpr (decltype(zero)::value) acc[i][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
          }
        return;
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float sc[4];
#pragma unroll
        for (int P = 0; P < 4; ++P) {
          const int c = nib_col<SEQ>(4 * h + P);
          const uint16_t sb = (uint16_t)(s4[c >> 1] >> (16 * (c & 1)));
          sc[P] = SBF ? bf_bits2f(sb) : h_bits2f(sb);
        }
        const HalfCoef hc = half_coef<T>(sc, zwc, 4 * h);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          if constexpr (ONE) {
            float tv[4] = {tot1[4 * h], tot1[4 * h + 1], tot1[4 * h + 2], tot1[4 * h + 3]};
            const float av[4] = {acc[4 * h][mt][0], acc[4 * h + 1][mt][0], acc[4 * h + 2][mt][0], acc[4 * h + 3][mt][0]};
            biased_terms<T>(tv, av, ax[mt][0], hc);
#pragma unroll
            for (int P = 0; P < 4; ++P) tot1[4 * h + P] = tv[P];
          } else {
            f32x4 tv[4] = {tot[4 * h][mt], tot[4 * h + 1][mt], tot[4 * h + 2][mt], tot[4 * h + 3][mt]};
            const f32x4 av[4] = {acc[4 * h][mt], acc[4 * h + 1][mt], acc[4 * h + 2][mt], acc[4 * h + 3][mt]};
            biased_terms<T>(tv, av, ax[mt], hc);
#pragma unroll
            for (int P = 0; P < 4; ++P) tot[4 * h + P][mt] = tv[P];
          }
        }
      }
      if constexpr (decltype(zero)::value) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          ax[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[i][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
    };
    auto prep = [&](int slot) {
      if constexpr (BIASED) zwc = sz[slot].zw;
      else
#pragma unroll
        for (int i = 0; i < 8; ++i) zm[i] = zero_magic(i & 1, (sz[slot].zw >> (4 * i)) & 0xF);
      s4 = sz[slot].s4;
    };

#pragma unroll
    for (int u = 0; u < D; ++u) issue(u, true);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (XL) {
      // this wave's DMA (issued before the ring) has landed once no more than the ring's loads
      // (two weight pieces, the scales and the zeros per unit) are in flight; the barrier then
      // covers every wave's
      AWQ_WAIT_VMCNT(D * (ZP ? 4 : 3));
      __syncthreads();
    }
    static_assert(D == 2 && (SPG == 1 || SPG % D == 0), "");
    constexpr bool kGroupLoop = SPG > 1;
    if (kGroupLoop && (w0 % SPG) == 0 && (nunits % SPG) == 0) {
      // whole groups (the usual case): one group per iteration, its first unit in slot 0, so
      // the MFMAs of that unit start from zero and nothing but tot is carried between groups
      for (int done = 0; done < nunits; done += SPG) {
        prep(0);
#pragma unroll
        for (int u = 0; u < SPG; ++u) {
          if (u == 0) compute(0, std::true_type{}, STREAM);
          else compute(u % D, std::false_type{}, STREAM);
          __builtin_amdgcn_sched_barrier(0);
          issue(u % D, false, STREAM);
          __builtin_amdgcn_sched_barrier(0);
        }
        flush(std::false_type{});
      }
    } else {
      // shares that start or end inside a group; with one k-step per group every unit is a
      // whole group (prepared, started from zero and scaled at once)
      int cks = w0;
      int g_cur = -1;
      for (int done = 0; done < nunits; done += D) {
#pragma unroll
        for (int u = 0; u < D; ++u) {
          if (done + u < nunits) {  // wave-uniform: the last turn may hold fewer units
            if constexpr (SPG == 1) {
              prep(u);
              compute(u, std::true_type{});
              flush(std::false_type{});
            } else {
              const int g = cks++ / SPG;
              if (g != g_cur) {
                if (g_cur >= 0) flush(std::true_type{});
                g_cur = g;
                prep(u);
              }
              compute(u, std::false_type{});
            }
          }
          __builtin_amdgcn_sched_barrier(0);
          issue(u, false);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      if (SPG > 1 && g_cur >= 0) flush(std::false_type{});  // the last group
    }
  } else if constexpr (XL) {
    AWQ_WAIT_VMCNT0();  // no ring: wait for this wave's DMA alone
    __syncthreads();
  }

  const int M = p.M;
  const int tile_floats = M * 128;  // one partial: [M, 128] fp32 (M = 1 in a row-exact launch)
  // partial (t, part): [M][128] floats, columns relative to the tile
  const __amdgpu_buffer_rsrc_t prs = make_rsrc(p.partial, (uint32_t)wk.tiles * (uint32_t)S * (uint32_t)tile_floats * 4u);
  const uint32_t tbase = (uint32_t)t * (uint32_t)S * (uint32_t)tile_floats * 4u;
  const uint32_t pbase = tbase + (uint32_t)part * (uint32_t)tile_floats * 4u;

  // ---- the waves' sums meet in LDS: lane (q, r) holds, for accumulator [i][mt] element v,
  // token mt*16 + 4q + v of column 8 r + nib_col(i); every wave parks its real tokens, then
  // each output is summed over the waves in wave order (fixed, so results are reproducible).
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int v = 0; v < (ONE ? 1 : 4); ++v) {
      const int m = mt * 16 + 4 * q + v;
      if (m >= M) continue;
      float o[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) o[c] = ONE ? tot1[col_nib<SEQ>(c)] : tot[col_nib<SEQ>(c)][mt][v];
      float* dst = &red[(wave * MROWS + m) * 128 + 8 * r];
      *(f32x4*)dst = f32x4{o[0], o[1], o[2], o[3]};
      *(f32x4*)(dst + 4) = f32x4{o[4], o[5], o[6], o[7]};
    }
  __syncthreads();
  const int ncols = min(128, p.N - t * 128);
  if (S == 1 && p.gate_act) {
    // gated epilogue: column j < 64 of the tile is a gate sum, 64 + j the matching up sum
    for (int o = tid; o < M * 64; o += NWV * 64) {
      const int m = o >> 6, col = o & 63;
      float g = red[m * 128 + col], u = red[m * 128 + 64 + col];
#pragma unroll
      for (int w = 1; w < NWV; ++w) {
        g += red[(w * MROWS + m) * 128 + col];
        u += red[(w * MROWS + m) * 128 + 64 + col];
      }
      const int oc = t * 64 + col;
      if (oc < p.n_out) p.c[(int64_t)m * p.ldc + oc] = to_bits<T>(gated_act(g, p.gate_act - 1) * u);
    }
    return;
  }
  for (int o = tid; o < M * 128; o += NWV * 64) {
    const int m = o >> 7, col = o & 127;
    float sum = red[m * 128 + col];
#pragma unroll
    for (int w = 1; w < NWV; ++w) sum += red[(w * MROWS + m) * 128 + col];
    if (S == 1) {
      if (col < ncols) {
        if (p.bias) sum += load_bias(p.bias, p.bias_dtype, t * 128 + col);
        p.c[(int64_t)m * p.ldc + t * 128 + col] = to_bits<T>(sum);
      }
    } else {
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, sum), prs, (int)(pbase + 4u * (uint32_t)o), 0,
                                            kDeviceCoherent);
    }
  }
  if (S == 1) return;
  __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores have completed (device scope)
  __syncthreads();                // ... and every thread's
  // The arrival count is an agent-scope release: it orders the block's partials (every wave's,
  // complete at the barrier above) before the count.  The block that arrives last then takes
  // an agent-scope acquire fence, which orders every other block's partials (their counts are
  // in the release sequence its increment read from) before its reads -- by the memory model
  // rather than by the cache-policy bits alone, which the partial stores and loads keep, so no
  // line of the partials is served stale from another XCD's L2.  On gfx950 the release writes
  // back this XCD's L2 and the acquire invalidates it; an acquire-release count in every block
  // cost 0.7 - 1.8 us per launch against relaxed counts, this form 0.3 - 0.6 us (M = 16,
  // N = 6144: 9.20 relaxed, 10.52 acquire-release, 9.77 this form).
  if (tid == 0) {
    s_last = __hip_atomic_fetch_add(&p.counters[t], 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT) == S - 1;
    if (s_last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
  __syncthreads();
  if (!s_last) return;
  // the last of the S blocks of tile t sums the partials in split (k) order, adds the bias
  // and writes the output (all threads of the block)
  const uint32_t pstride = (uint32_t)tile_floats * 4u;  // bytes between splits
  if (p.gate_act) {
    // gated epilogue: gate columns 2ch, 2ch + 1 and their up columns 64 further on, each
    // summed over the splits in split order like the plain output
    for (int idx = tid; idx < M * 32; idx += NWV * 64) {
      const int m = idx >> 5, ch = idx & 31;
      const uint32_t off = tbase + ((uint32_t)m * 128u + 2u * (uint32_t)ch) * 4u;
      f32x2 g = {0.f, 0.f}, u = {0.f, 0.f};
      for (int c0 = 0; c0 < S; c0 += 4) {
        f32x2 vg[4], vu[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t o = (c0 + e < S) ? off + (uint32_t)(c0 + e) * pstride : 0x80000000u;
          vg[e] = __builtin_bit_cast(f32x2, __builtin_amdgcn_raw_buffer_load_b64(prs, (int)o, 0, kDeviceCoherent));
          vu[e] = __builtin_bit_cast(f32x2, __builtin_amdgcn_raw_buffer_load_b64(prs, (int)(o + 256u), 0, kDeviceCoherent));
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          g += vg[e];
          u += vu[e];
        }
      }
      const int oc = t * 64 + 2 * ch;
      uint16_t* dst = p.c + (int64_t)m * p.ldc + oc;
      if (oc < p.n_out) dst[0] = to_bits<T>(gated_act(g[0], p.gate_act - 1) * u[0]);
      if (oc + 1 < p.n_out) dst[1] = to_bits<T>(gated_act(g[1], p.gate_act - 1) * u[1]);
    }
    if (tid == 0) __hip_atomic_store(&p.counters[t], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  const int nh = ncols >> 1;  // float2 chunks per row
  for (int idx = tid; idx < M * nh; idx += NWV * 64) {
    const int m = idx / nh, ch = idx - m * nh;
    const uint32_t off = tbase + ((uint32_t)m * 128u + 2u * (uint32_t)ch) * 4u;
    // splits in groups of 8 whose loads are in flight together; slots past S read as zero
    // (out of the buffer range), and the sum runs in split order
    f32x2 sum = {0.f, 0.f};
    for (int c0 = 0; c0 < S; c0 += 8) {
      f32x2 v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t o = (c0 + e < S) ? off + (uint32_t)(c0 + e) * pstride : 0x80000000u;
        v[e] = __builtin_bit_cast(f32x2, __builtin_amdgcn_raw_buffer_load_b64(prs, (int)o, 0, kDeviceCoherent));
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) sum += v[e];
    }
    const int col = t * 128 + 2 * ch;
    if (p.bias) {
      sum[0] += load_bias(p.bias, p.bias_dtype, col);
      sum[1] += load_bias(p.bias, p.bias_dtype, col + 1);
    }
    *(uint32_t*)(p.c + (int64_t)m * p.ldc + col) = pack2<T>(sum[0], sum[1]);
  }
  if (tid == 0) __hip_atomic_store(&p.counters[t], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace awq

namespace awq_host {
using namespace awq;

// M == 1 needs few enough registers to run blocks of 16 waves at four per SIMD, which hides
// more of the memory latency; more tokens run 8 waves at two per SIMD, whose registers leave
// room for the whole-group loop (measured faster than 16 waves without it).
// Activation slices up to this many bytes per block are staged in LDS (M == 1, stream layout).
constexpr uint32_t kDecodeXlMax = 49152;

template <int MT, bool SEQ, bool ZP, typename T, bool SBF, bool STREAM, bool ONE, bool XL>
inline void launch_x(const GemmArgs& a, const DecodePlan& s, uint32_t shmem, hipStream_t st) {
  const DecodeWork wk{s.tiles, s.ksteps, s.splits, s.per};
  constexpr int NWV = ONE ? 16 : 8, OCC = ONE ? 4 : 2;
  const dim3 grid((unsigned)(s.blocks * (a.rows > 1 ? a.rows : 1))), block(NWV * 64);
  const int spg = a.G / 32;
  if (spg == 4)
    hipLaunchKernelGGL((decode_kn_kernel<MT, NWV, 2, 4, SEQ, ZP, T, SBF, STREAM, ONE, OCC, XL>), grid, block, shmem, st, a, wk);
  else if (spg == 2)
    hipLaunchKernelGGL((decode_kn_kernel<MT, NWV, 2, 2, SEQ, ZP, T, SBF, STREAM, ONE, OCC, XL>), grid, block, shmem, st, a, wk);
  else
    hipLaunchKernelGGL((decode_kn_kernel<MT, NWV, 2, 1, SEQ, ZP, T, SBF, STREAM, ONE, OCC, XL>), grid, block, shmem, st, a, wk);
}

template <int MT, bool SEQ, bool ZP, typename T, bool SBF, bool STREAM, bool ONE>
inline void launch_t(const GemmArgs& a, const DecodePlan& s, hipStream_t st) {
  if constexpr (ONE && STREAM) {
    const uint32_t xbytes = (uint32_t)((s.per + 15) / 16) * 1024u;  // whole DMA instructions
    if (xbytes <= kDecodeXlMax) {
      launch_x<MT, SEQ, ZP, T, SBF, STREAM, ONE, true>(a, s, xbytes, st);
      return;
    }
  }
  launch_x<MT, SEQ, ZP, T, SBF, STREAM, ONE, false>(a, s, 0, st);
}

// ONE selects the M == 1 instantiation (the f16 paths only; the others use the general one)
template <bool SEQ, bool ZP, typename T, bool SBF, bool STREAM, bool HAS_ONE>
inline bool launch_sel(const GemmArgs& a, const DecodePlan& s, hipStream_t st) {
  if (s.mt == 2) launch_t<2, SEQ, ZP, T, SBF, STREAM, false>(a, s, st);
  else if (HAS_ONE && a.M == 1) launch_t<1, SEQ, ZP, T, SBF, STREAM, HAS_ONE>(a, s, st);
  else launch_t<1, SEQ, ZP, T, SBF, STREAM, false>(a, s, st);
  return true;
}

}  // namespace awq_host
