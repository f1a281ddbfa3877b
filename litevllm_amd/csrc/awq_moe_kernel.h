// Grouped AWQ W4A16 mixture-of-experts kernels for gfx950: the role of
// gemma4_moe_int4_prefill_grouped / _fused (vllm/kernels/triton/gemma4_moe_int4.py:2330-2584,
// kernels at 626-760 and 894-1030) and of the expert loop of fused_moe
// (vllm/model_executor/layers/fused_moe/fused_moe.py:4-77), for zero-point or symmetric int4
// experts with any group size 32 / 64 / 128.
//
//  * route lists (moe_align_kernel): for each expert, the indices r = token * top_k + j of
//    the routes that chose it, in route order (the stable sort by expert id of the reference
//    wrapper, gemma4_moe_int4.py:2520-2523), plus the count.
//  * gate_up (moe_gemm_kernel<0>): grid (column tile, expert).  An expert's gate_up weight
//    [H, 2I] is read in the stream layout with its tiles pairing 8 gate words with the 8 up
//    words of the same columns, so one MFMA operand set yields gate and up together.  The
//    block's waves split K; the sums meet in LDS in a fixed order; the epilogue computes
//    act(gate) * up * route_weight in fp32 and rounds once to the activation dtype -- the
//    intermediate the reference keeps in x.dtype (gemma4_moe_int4.py:748-760).
//  * down (moe_gemm_kernel<1>): the same structure over the intermediate rows, writing one fp32
//    row per route.
//  * combine (moe_combine_kernel): out[t] = round(sum_j y[t * top_k + j]) in j order, fp32.
//
// Every route row is computed independently of which other rows share its tile, and every sum
// runs in a fixed order, so results are bitwise reproducible.
#pragma once

#include "awq_common.h"
#include "awq_launch.h"

namespace awq {

// Packed word of the expert weight held by lane r of tile t: with gate/up pairing (half =
// I / 8 > 0) lanes 0-7 hold gate words 8t .. 8t+7 and lanes 8-15 the up words half + 8t ..;
// without, lanes hold words 16t .. 16t+15.  -1 past the end (zero weights, never stored).
__host__ __device__ inline int moe_word(int t, int r, int half, int NW) {
  if (half > 0) {
    const int w = 8 * t + (r & 7);
    if (w >= half) return -1;
    return r < 8 ? w : half + w;
  }
  const int w = 16 * t + r;
  return w < NW ? w : -1;
}

struct MoeArgs {
  const uint16_t* a;   // gate_up: x [T, lda]; down: the intermediate [R, lda = I]
  const uint32_t* qw;  // stream-packed expert stack [E][tiles][K/32][2048 B]
  const uint16_t* sc;  // scales [E][K/G][N]
  const uint32_t* qz;  // zeros [E][K/G][N/8] (AutoAWQ order) or null (symmetric, z = 8)
  const int* lists;    // route lists [E][R], or null: each block collects its expert's routes
  const int* counts;   // routes per expert [E]   from ids (R <= kMoeScanMaxR)
  const void* ids;     // expert ids [R], int32 or int64 (id64)
  int id64;
  const void* rw;      // route weights [R] (gate_up only)
  void* out;           // gate_up: [R][ldo] act dtype; down: [R][ldo] fp32
  int64_t lda, ldo;
  int R, topk, K, N, G, half, tiles, rows_a;
  int rw_dtype, act_kind;
};

// Largest route count whose route lists the stream kernels collect themselves.
constexpr int kMoeScanMaxR = 1024;

__device__ __forceinline__ float load_route_weight(const void* rw, int dtype, int r) {
  if (dtype == AWQ_DTYPE_F16) return h_bits2f(((const uint16_t*)rw)[r]);
  if (dtype == AWQ_DTYPE_BF16) return bf_bits2f(((const uint16_t*)rw)[r]);
  return ((const float*)rw)[r];
}

// MT: 16-route tiles per wave group.  SBF: scales are bf16 (fp16 otherwise).  Like the decode
// kernel, the MFMAs multiply the activations by the exact integers q - z and each group's
// fp32 sum is scaled once by the group's scale, so the weights enter unrounded -- the
// reference's int4 kernels do the same, x * (q - 8) * s in fp32 (gemma4_moe_int4.py:736-742).
template <int MODE, int MT, int D, int SPG, bool ZP, typename T, bool SBF, int NWV>
__global__ void __launch_bounds__(64 * NWV) __attribute__((amdgpu_waves_per_eu(MT == 1 ? 4 : 2, MT == 1 ? 4 : 2)))
moe_gemm_kernel(const MoeArgs p) {
  constexpr int NACC = 8 * MT;
  constexpr int CH = NACC < 16 ? NACC : 16;
  static_assert(NACC % CH == 0, "");
  static_assert(D == 2 && (SPG == 1 || SPG % D == 0), "");
  __shared__ f32x4 red[(NWV / 2) * CH * 64];
  __shared__ int s_list[kMoeScanMaxR];  // the expert's routes, collected from the ids
  __shared__ int s_wc[NWV];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q = lane >> 4, r = lane & 15;
  const int t = blockIdx.x, e = blockIdx.y;

  const int KS = p.K >> 5;
  const int NW = p.N >> 3;
  const int ngroups = p.K / p.G;
  const int* list = p.lists + (int64_t)e * p.R;
  const uint32_t stream_bytes = (uint32_t)p.tiles * (uint32_t)KS * 2048u;
  const char* wbase = (const char*)p.qw + (int64_t)e * stream_bytes;
  // weight units of a ring slot: 2 x 16 bytes per lane of the unit's 2 KiB run (zeros past the
  // wave's last unit: an empty descriptor, no memory traffic)
  uint32_t raw[D][8];
  auto load_w = [&](int slot, int ks, bool past) {
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(wbase, past ? 0u : stream_bytes);
    const int kbase = (int)(((uint32_t)t * (uint32_t)KS + (uint32_t)ks) * 2048u);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const u32x4 v = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(wrs, (int)((uint32_t)lane * 16u), kbase + 1024 * i, kStreamNT));
#pragma unroll
      for (int c = 0; c < 4; ++c) raw[slot][4 * i + c] = v[c];
    }
  };
  // The first round's weights are requested before the route count is known, for the
  // one-group split (every wave on the first 16 * MT routes, K split over the block): the split
  // of every expert with at most 16 * MT routes.  What the route count depends on is requested
  // first, so that waiting for it does not wait for the weights: the ids (the block collects
  // its expert's routes) or the first round's route rows (route lists given).
  const bool scan = p.lists == nullptr;  // kernel-uniform
  constexpr int SPT = kMoeScanMaxR / (64 * NWV);  // ids per thread
  int idv[SPT];
  int pre_rt[MT];
  auto load_first_weights = [&]() __attribute__((always_inline)) {
    const int ks0 = KS * wave / NWV, n = KS * (wave + 1) / NWV - ks0;
#pragma unroll
    for (int u = 0; u < D; ++u) load_w(u, ks0 + u, u >= n);
    __builtin_amdgcn_sched_barrier(0);
  };
  if (scan) {
    // int64 ids: the low word (the value for every id below 2^31), as the route lists kernel
    const uint32_t stride = p.id64 ? 8u : 4u;
    const __amdgpu_buffer_rsrc_t irs = make_rsrc(p.ids, (uint32_t)p.R * stride);
#pragma unroll
    for (int u = 0; u < SPT; ++u) {
      const int i = u * 64 * NWV + tid;
      const int v = (int)__builtin_amdgcn_raw_buffer_load_b32(irs, (int)((uint32_t)i * stride), 0, 0);
      idv[u] = i < p.R ? v : -1;
    }
    load_first_weights();
  } else {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) pre_rt[mt] = mt * 16 + r < p.R ? list[mt * 16 + r] : -1;
    load_first_weights();
  }
  int count;
  if (scan) {
    // routes whose id is e, in route order (the order the route lists hold)
    int c = 0;
#pragma unroll
    for (int u = 0; u < SPT; ++u) {
      if (u * 64 * NWV < p.R) {  // block-uniform
        const bool hit = idv[u] == e;
        const uint64_t m = __ballot(hit);
        if (lane == 0) s_wc[wave] = __popcll(m);
        __syncthreads();
        int off = c, tot = c;
#pragma unroll
        for (int w = 0; w < NWV; ++w) {
          off += w < wave ? s_wc[w] : 0;
          tot += s_wc[w];
        }
        if (hit) s_list[off + __popcll(m & ((1ull << lane) - 1ull))] = u * 64 * NWV + tid;
        __syncthreads();  // the list is complete, and s_wc is read before the next round writes it
        c = tot;
      }
    }
    count = __builtin_amdgcn_readfirstlane(c);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) pre_rt[mt] = mt * 16 + r < count ? s_list[mt * 16 + r] : -1;
  } else {
    count = p.counts[e];
  }
  if (count == 0) return;  // whole block
  auto route_at = [&](int m) -> int { return scan ? s_list[m] : list[m]; };
  const uint16_t* sbase = p.sc + (int64_t)e * ngroups * p.N;
  const void* zbase = ZP ? (const void*)(p.qz + (int64_t)e * ngroups * NW) : (const void*)p.sc;
  const uint32_t s_bytes = (uint32_t)ngroups * (uint32_t)p.N * 2u;
  const uint32_t z_bytes = ZP ? (uint32_t)ngroups * (uint32_t)NW * 4u : 0u;
  const uint32_t x_bytes = (uint32_t)((uint64_t)p.rows_a * (uint64_t)p.lda * 2u);
  const int word = moe_word(t, r, p.half, NW);
  const uint32_t wc = word < 0 ? 0u : (uint32_t)word;  // padding lanes: word 0's constants, zero weights
  const MagicK mk = magic_consts();
  const BiasK bk = bias_consts<T>();
  const u32x4 ones = {ones2<T>(), ones2<T>(), ones2<T>(), ones2<T>()};
  // biased operands (see biased_operand) where they need fewer instructions than the exact
  // integers q - z: several k-steps per group of one route tile, and bf16
  constexpr bool BIASED = (SPG >= 2 && MT == 1) || (!std::is_same<T, f16>::value && !(MT == 2 && SPG == 1));

  // one round per 16 * MT * (wave groups) routes; the first is its own copy of the code, so
  // that the waits of its first loads see only what was requested before it
  auto run_round = [&](const int base, auto first_t) __attribute__((always_inline)) -> int {
    constexpr bool FIRST = decltype(first_t)::value;
    // wave groups of 16 * MT rows; the waves of a group split K
    const int left = count - base;
    int ng = 1;
    while (ng < NWV && ng * 16 * MT < left) ng <<= 1;
    const int wpg = NWV / ng;
    const int gi = wave / wpg, ki = wave - gi * wpg;
    const int m0 = base + gi * 16 * MT;
    const bool active = m0 < count;  // wave-uniform
    const int ks0 = KS * ki / wpg, ks1 = KS * (ki + 1) / wpg;
    const int nunits = ks1 - ks0;

    f32x4 acc[8][MT];  // the current group's sums, integer (or biased) weights
    f32x4 ax[MT];      // the current group's activation sums (biased operands)
    f32x4 tot[8][MT];  // the scaled sums of the groups done
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      ax[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i][mt] = tot[i][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    // the first round of the one-group split: its weights and rows are in flight already
    const bool pre = FIRST && ng == 1;  // block-uniform
    if (active && nunits > 0) {
      // the activation operand: route row r of each 16-route tile, 8 k per lane
      uint32_t x_off[MT];
      // (the divisor is re-read each round, so that its reciprocal is not held across the
      // k-step loop)
      int topk = p.topk;
      asm volatile("" : "+s"(topk));
      int ln = lane;
      asm volatile("" : "+v"(ln));
      auto row_off = [&](int rt) -> uint32_t {
        const uint32_t arow = MODE == 0 ? (uint32_t)rt / (uint32_t)topk : (uint32_t)rt;
        return rt < 0 ? 0x80000000u : arow * (uint32_t)p.lda * 2u + 16u * (uint32_t)(ln >> 4);
      };
      // two branches, each using its rows inside: the wait for a list read issued after the
      // weights (later rounds) must not apply to the first round, whose rows came first
      if (pre) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) x_off[mt] = row_off(mt * 16 + r < count ? pre_rt[mt] : -1);
      } else if (scan) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int m = m0 + mt * 16 + r;
          x_off[mt] = row_off(m < count ? s_list[m] : -1);
        }
      } else {
        const __amdgpu_buffer_rsrc_t lrs = make_rsrc(list, (uint32_t)p.R * 4u);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int m = m0 + mt * 16 + r;
          const int rt = m < count ? (int)__builtin_amdgcn_raw_buffer_load_b32(lrs, (int)(4u * (uint32_t)m), 0, 0) : -1;
          x_off[mt] = row_off(rt);
          asm volatile("" : "+v"(x_off[mt]));
        }
      }
      u32x4 xr[D][MT];
      WordSZ sz[D];
      uint32_t zm[8];  // biased zeros of the current group (exact integer operands)
      uint32_t zwc;    // zero word of the current group (biased operands)
      u32x4 s4;        // scales of the current group (the word's 8 columns, raw 16-bit values)
      // past the wave's last unit the ring's refills go through empty descriptors (zeros,
      // no memory traffic), so every ring turn is a whole one
      int iks = ks0, ileft = nunits;
      // scales and zeros only where a group starts or in the first turn (prep reads no other
      // slot's); the single-tile kernel keeps per-unit loads (its 128 registers have no room
      // to hold a slot's constants across turns)
      auto issue = [&](int slot, bool first_turn, bool with_w = true) {
        const int ks = iks;
        const bool past = ileft <= 0;
        ++iks;
        --ileft;
        const __amdgpu_buffer_rsrc_t xrs = make_rsrc(p.a, past ? 0u : x_bytes);
        const __amdgpu_buffer_rsrc_t srs = make_rsrc(sbase, past ? 0u : s_bytes);
        const __amdgpu_buffer_rsrc_t zrs = make_rsrc(zbase, past ? 0u : z_bytes);
        if (with_w) load_w(slot, ks, past);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          xr[slot][mt] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, (int)x_off[mt], ks * 64, 0));
        if (first_turn || (ks & (SPG - 1)) == 0 || MT == 1) {  // wave-uniform
          const int g = ks / SPG;
          sz[slot].s4 = __builtin_bit_cast(
              u32x4, __builtin_amdgcn_raw_buffer_load_b128(srs, (int)(16u * wc), (int)((uint32_t)g * (uint32_t)p.N * 2u), 0));
          sz[slot].zw = ZP ? __builtin_amdgcn_raw_buffer_load_b32(zrs, (int)(4u * wc), (int)((uint32_t)g * (uint32_t)NW * 4u), 0)
                           : 0x88888888u;
        }
      };
      // FRESH: the group's first unit (its MFMAs start from zero)
      auto compute = [&](int slot, auto fresh) {
        constexpr bool FRESH = decltype(fresh)::value;
        uint32_t mlo[4], mhi[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {  // rows arrive paired (moe_pack_stream_kernel)
          mlo[v] = raw[slot][v];
          mhi[v] = raw[slot][4 + v];
        }
#define AWQ_MOE_NIB(I)                                                                          \
        {                                                                                       \
          const u32x4 op = BIASED ? biased_operand<I, T>(mlo, mhi, bk) : int_operand<I, T>(mlo, mhi, zm[I], mk); \
          _Pragma("unroll") for (int mt = 0; mt < MT; ++mt)                                     \
              acc[I][mt] = MfmaOp<T>::run(xr[slot][mt], op, FRESH ? f32x4{0.f, 0.f, 0.f, 0.f} : acc[I][mt]); \
        }
        AWQ_MOE_NIB(0) AWQ_MOE_NIB(1) AWQ_MOE_NIB(2) AWQ_MOE_NIB(3)
        AWQ_MOE_NIB(4) AWQ_MOE_NIB(5) AWQ_MOE_NIB(6) AWQ_MOE_NIB(7)
#undef AWQ_MOE_NIB
        if constexpr (BIASED)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            ax[mt] = MfmaOp<T>::run(xr[slot][mt], ones, FRESH ? f32x4{0.f, 0.f, 0.f, 0.f} : ax[mt]);
      };
      // tot += acc * scale of the group just finished (ZERO: acc restarts from zero)
      auto flush = [&](auto zero) {
        if constexpr (BIASED) {
          flush_biased<T, SBF>(tot, acc, ax, s4, zwc);
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const int c = nib_col<false>(i);
            const uint16_t sb = (uint16_t)(s4[c >> 1] >> (16 * (c & 1)));
            const float sf = SBF ? bf_bits2f(sb) : h_bits2f(sb);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) tot[i][mt] += acc[i][mt] * sf;
          }
        }
        if constexpr (decltype(zero)::value)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            ax[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[i][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
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
      for (int u = 0; u < D; ++u) issue(u, true, !pre);
      __builtin_amdgcn_sched_barrier(0);
      // (one token tile runs without it: the extra loop would cost the registers that let
      // four waves share a SIMD)
      constexpr bool kGroupLoop = SPG > 1 && MT > 1;
      if (kGroupLoop && (ks0 % SPG) == 0 && (nunits % SPG) == 0) {
        // whole groups: one group per iteration, its first unit in slot 0
        for (int done = 0; done < nunits; done += SPG) {
          prep(0);
#pragma unroll
          for (int u = 0; u < SPG; ++u) {
            if (u == 0) compute(0, std::true_type{});
            else compute(u % D, std::false_type{});
            __builtin_amdgcn_sched_barrier(0);
            issue(u % D, false);
            __builtin_amdgcn_sched_barrier(0);
          }
          flush(std::false_type{});
        }
      } else {
        int cks = ks0, g_cur = -1;
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
        if (SPG > 1 && g_cur >= 0) flush(std::false_type{});
      }
    }

    // ---- the group's sums meet in LDS, fixed tree order ----
    const int hslots = wpg >> 1;  // reduction slots per group
#pragma unroll
    for (int c0 = 0; c0 < NACC; c0 += CH) {
      for (int half = hslots; half >= 1; half >>= 1) {
        if (ki >= half && ki < 2 * half) {
#pragma unroll
          for (int c = 0; c < CH; ++c)
            red[((gi * hslots + ki - half) * CH + c) * 64 + lane] = tot[(c0 + c) / MT][(c0 + c) % MT];
        }
        __syncthreads();
        if (ki < half) {
#pragma unroll
          for (int c = 0; c < CH; ++c) tot[(c0 + c) / MT][(c0 + c) % MT] += red[((gi * hslots + ki) * CH + c) * 64 + lane];
        }
        __syncthreads();
      }
    }

    // ---- epilogue: the group's first wave holds the sums ----
    // lane (q, r), accumulator [i][mt] element v: route row m0 + 16 mt + 4q + v, tile word r,
    // column nib_col(i) of that word
    if (ki == 0 && active) {
      // the lane's row and word taken afresh (nothing derived from them is held across the
      // k-step loop)
      int ln = lane;
      asm volatile("" : "+v"(ln));
      const int q = ln >> 4, r = ln & 15;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int m = m0 + mt * 16 + 4 * q + v;
          const int rt = m < count ? route_at(m) : -1;
          if constexpr (MODE == 0) {
            // the up sums of the gate columns sit 8 lanes higher (tile words 8 .. 15).  Lane
            // r < 8 finishes columns 0..3 of gate word 8 t + r and lane r + 8 columns 4..7 of
            // the same word: per column pair, two row rotations by 8 that each write one half
            // of the row (DPP bank mask; the other half keeps its own value) give every lane
            // the gate and the up sum of its column
            float gt[4], ut[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              float a = tot[col_nib<false>(j)][mt][v], b = tot[col_nib<false>(4 + j)][mt][v];
              asm volatile("" : "+v"(a), "+v"(b));
              gt[j] = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, a), __builtin_bit_cast(int, b), 0x128, 0xF, 0xC, false));
              ut[j] = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, b), __builtin_bit_cast(int, a), 0x128, 0xF, 0x3, false));
            }
            const int gw = 8 * t + (r & 7);  // gate word
            if (rt >= 0 && gw < p.half) {
              const float wgt = load_route_weight(p.rw, p.rw_dtype, rt);
              float h[4];
#pragma unroll
              for (int j = 0; j < 4; ++j) h[j] = gated_act(gt[j], p.act_kind) * ut[j] * wgt;
              *(u32x2*)((uint16_t*)p.out + (int64_t)rt * p.ldo + 8 * gw + (r & 8) / 2) =
                  u32x2{pack2<T>(h[0], h[1]), pack2<T>(h[2], h[3])};
            }
          } else {
            float o[8];
#pragma unroll
            for (int c = 0; c < 8; ++c) o[c] = tot[col_nib<false>(c)][mt][v];
            const int w = 16 * t + r;
            if (rt >= 0 && w < NW) {
              float* dst = (float*)p.out + (int64_t)rt * p.ldo + 8 * w;
              *(f32x4*)dst = f32x4{o[0], o[1], o[2], o[3]};
              *(f32x4*)(dst + 4) = f32x4{o[4], o[5], o[6], o[7]};
            }
          }
        }
      }
    }
    return base + ng * 16 * MT;
  };
  int base = run_round(0, std::true_type{});
  while (base < count) base = run_round(base, std::false_type{});
}

}  // namespace awq

namespace awq_host {
using namespace awq;

// waves per block: the 944-1024 blocks of a decode batch's grid (tiles x experts) fit the chip
// at once with four-wave blocks (four blocks per CU at one 16-route tile), and each wave
// streams twice the k-steps of an eight-wave block
constexpr int kMoeStreamWaves = 4;

// grid (column tiles, experts); the group size picks the k-steps per group
template <int MODE, int MT, bool ZP, typename T, bool SBF>
inline void launch_moe_gemm_t(const MoeArgs& a, int E, hipStream_t st) {
  const dim3 grid((unsigned)a.tiles, (unsigned)E);
  const int spg = a.G / 32;
  if (spg == 4)
    hipLaunchKernelGGL((moe_gemm_kernel<MODE, MT, 2, 4, ZP, T, SBF, kMoeStreamWaves>), grid, dim3(64 * kMoeStreamWaves), 0, st, a);
  else if (spg == 2)
    hipLaunchKernelGGL((moe_gemm_kernel<MODE, MT, 2, 2, ZP, T, SBF, kMoeStreamWaves>), grid, dim3(64 * kMoeStreamWaves), 0, st, a);
  else
    hipLaunchKernelGGL((moe_gemm_kernel<MODE, MT, 2, 1, ZP, T, SBF, kMoeStreamWaves>), grid, dim3(64 * kMoeStreamWaves), 0, st, a);
}

// grouped MFMA kernels for many routes per expert (awq_moe_mfma.hip, awq_moe_mfma_down.hip);
// both K dims % 64 == 0
void launch_moe_mfma(const awq::MoeArgs& gu, const awq::MoeArgs& dn, int E, bool zp, int act, int sbf,
                     hipStream_t st);
void launch_moe_tile_down(const awq::MoeArgs& dn, int E, bool zp, int act, int sbf, hipStream_t st);
// bf16 activations or bf16 scales (awq_moe_misc.hip); false if the dtype is not provided
bool launch_moe_misc(const awq::MoeArgs& gu, const awq::MoeArgs& dn, int E, bool zp, int act, int sbf,
                     hipStream_t st);
}  // namespace awq_host
