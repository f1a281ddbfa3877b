// Grouped MoE GEMMs for many routes per expert (prefill-sized batches) on gfx950: the work of
// moe_gemm_kernel (awq_moe_kernel.h) restructured so that each dequantized weight operand feeds
// up to six 16-route MFMA tiles (moe_tile_kernel).  Instantiated by awq_moe_mfma.hip (gate_up)
// and awq_moe_mfma_down.hip (down).
#pragma once

#include "awq_moe_kernel.h"

namespace awq {

// routes per row tile (six 16-route MFMA tiles), k per stage (one MFMA k-step), stream tiles
// per block, stage slots
constexpr int kTBM = 96, kTBK = 32, kTST = 4, kTPD = 5;

// Row tile t of the grid: first every expert's full kTBM-route tiles (expert order), then
// every expert's last partial tile, so the heavy tiles are dispatched first.  Computed by one
// wave from the per-expert route counts, 64 experts per pass (one count per lane, prefix sums
// across the wave), so a block spends one round of count loads on it.  e = -1 past the end.
// have0: the lane's count of expert `lane` is already in cnt0 (the first 64 experts).
// The scan and the lane reads are DPP and readlane operations: shuffles routed through the LDS
// wait here behind the block's first weight DMAs landing in LDS (T = 512 gate_up 62.9 -> 60.3 us
// in a kernel-trace A/B on one box: two alternating runs each)
__device__ inline void moe_row_tile_wave(const int* counts, int E, int t, int& e, int& m0, int& rows, bool have0 = false,
                                         int cnt0 = 0) {
  const int lane = threadIdx.x & 63;
  e = -1;
  m0 = 0;
  rows = 0;
  // phase 0: full tiles, phase 1: partial tiles
  for (int phase = 0; phase < 2 && e < 0; ++phase) {
    int base = 0;
    for (int c0 = 0; c0 < E; c0 += 64) {
      const int ex = c0 + lane;
      const int cnt = (have0 && c0 == 0) ? cnt0 : (ex < E ? counts[ex] : 0);
      const int n = phase == 0 ? cnt / kTBM : (cnt % kTBM != 0 ? 1 : 0);
      const int incl = wave_incl_scan_i32(n);
      const int tot = __builtin_amdgcn_readlane(incl, 63);
      if (t < base + tot) {  // wave-uniform
        const uint64_t hit = __ballot(base + incl > t);
        const int l = __builtin_amdgcn_readfirstlane(__ffsll((long long)hit) - 1);
        const int excl = __builtin_amdgcn_readlane(incl - n, l);
        const int c = __builtin_amdgcn_readlane(cnt, l);
        e = c0 + l;
        if (phase == 0) {
          m0 = (t - base - excl) * kTBM;
          rows = kTBM;
        } else {
          rows = c % kTBM;
          m0 = c - rows;
        }
        break;
      }
      base += tot;
    }
    t -= base;
  }
}

// One block: one row tile of an expert's route list (up to 96 routes: six 16-route MFMA tiles)
// times kTST consecutive stream tiles (128 weight columns each), 8 waves: wave w owns stream
// tile w % 4 and K-half w / 4, so two waves share each SIMD (each with at least 32 independent
// accumulators at four token tiles, which keeps the MFMA pipe issuing) and one's memory and
// LDS waits are covered by the other's work.
//  * Per 32-row k-step a lane reads its 32-byte piece of the stream layout (one packed word
//    over 8 k-rows), pairs the rows, dequantizes each nibble position to one MFMA operand (the
//    exact magic-number dequant, (q - z) * s rounded once to the activation dtype) and
//    multiplies it into every token tile (v_mfma_f32_16x16x32): one dequant feeds up to six
//    MFMAs, and at T = 512 every expert's routes (about 64, at most 84 in the benchmark) fit one
//    row tile, so each weight is dequantized once per K-half wave and the grid is one block
//    per CU (a second, partial tile of an expert would start a second round of blocks).
//  * Everything a k-step needs comes into LDS by DMA four k-steps ahead (five slots): each
//    K-half's activation rows (gathered from the route rows, shared by its 4 waves) and each
//    wave's weight pieces, scales and zeros; the request's DMA instructions are spread over
//    the k-step's MFMAs.  One barrier per k-step: it marks the k-step's data complete and the
//    slot read in the previous k-step free for the next request.
//  * The route ids and weights of the tile sit in LDS, so the epilogue waits on no global load;
//    the activation comes from the hardware exp2 and reciprocal (gated_act_fast), rounded to
//    the activation dtype right after.
//  * The K-halves meet in LDS (fixed order: first half + second half), then lane (q, r) of the
//    first-half wave holds the 8 columns 8 w .. 8 w + 7 of its word w for rows 4 q .. 4 q + 3 of
//    each token tile, so the epilogue stores contiguous values per row: for gate_up lane r
//    (gate sums) and lane r + 8 (up sums of the same columns) trade halves through row
//    rotations by 8 lanes, each finishes 4 of the word's columns, and act(gate) * up *
//    route_weight is rounded once into the intermediate; down writes fp32 rows per route.
// fp32 sums; the intermediate is rounded once to the activation dtype and down writes fp32
// route rows, as in moe_gemm_kernel.  Every row is computed independently of its tile mates, so
// results are bitwise reproducible.
template <int MODE, bool ZP, typename T, bool FAST>
__global__ void __launch_bounds__(128 * kTST) moe_tile_kernel(const MoeArgs p, int scale_bf16, int E, int col_groups) {
  constexpr int BM = kTBM, BK = kTBK, PD = kTPD, NWV = 2 * kTST;
  constexpr int CPR = BK / 8;                 // 16-byte chunks per activation row (4)
  constexpr int A_INSTR = BM * CPR / 64;      // activation DMAs per K-half per k-step (6)
  constexpr int A_TWO = A_INSTR - kTST;       // waves of a half that issue two of them (2)
  static_assert(A_TWO > 0 && A_TWO <= kTST && A_INSTR * 64 == BM * CPR, "activation DMA split");
  // one slot (16-byte chunks): A [2 halves][BM rows][CPR], W [NWV][2 pieces][64 lanes],
  // S [NWV][16 words], Z [NWV][16] (uint32)
  constexpr int A_OFF = 0, W_OFF = A_OFF + 2 * BM * CPR, S_OFF = W_OFF + NWV * 2 * 64;
  constexpr int Z_OFF = S_OFF + NWV * 16, SLOT = Z_OFF + NWV * 16 / 4;
  constexpr uint32_t SLOT_BYTES = (uint32_t)SLOT * 16u;
  __shared__ u32x4 lds_all[PD * SLOT];
  __shared__ int s_rt[BM];
  __shared__ float s_w[BM];
  __shared__ int s_tile[4];
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) u32x4*)&lds_all[0];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int stl = wave & (kTST - 1), kh = wave / kTST;
  const int q = lane >> 4, r = lane & 15;

  // this block's column group and row tile: the column groups of one row tile run on one XCD
  // (the hardware deals blocks to the 8 XCDs round robin; the launch makes the row tiles a
  // multiple of 8), so they gather the tile's rows into that XCD's L2 once (T = 512: gate_up
  // 65.2 -> 64.4 us, down 40.0 -> 38.8 us, kernel-trace A/B on one box)
  int cg, t_tile;
  {
    const int b = (int)blockIdx.x, nrt = (int)gridDim.x / col_groups;
    if ((nrt & 7) == 0) {
      const int i = b >> 3;
      cg = i % col_groups;
      t_tile = (i / col_groups) * 8 + (b & 7);
    } else {
      cg = b % col_groups;
      t_tile = b / col_groups;
    }
  }
  const int KS = p.K >> 5;
  const int NW = p.N >> 3;
  const int ngroups = p.K / p.G;
  const int lg = __builtin_ctz((unsigned)p.G);  // the launcher takes power-of-two group sizes only
  const int st = cg * kTST + stl;              // this wave's stream tile
  const bool wave_on = st < p.tiles;
  const int word = wave_on ? moe_word(st, r, p.half, NW) : -1;
  const uint32_t wc = word < 0 ? 0u : (uint32_t)word;
  // K-halves in k-steps: the first half takes the odd one when there is one
  const int n0 = (KS + 1) >> 1;
  const int n_my = kh == 0 ? n0 : KS - n0;
  const int s_first = kh == 0 ? 0 : n0;  // first global k-step of this wave's half

  // ---- activation gather: DMA i (0..5) of a half fills its chunks 64 i + lane: row
  // 16 i + lane / 4, slot lane % 4, holding k-chunk slot ^ ((row / 2) & 3); wave (stl, kh)
  // issues DMA stl of its half, and waves stl < 2 also DMA 4 + stl ----
  const u32x4 ars = rsrc_words(p.a, (uint32_t)((uint64_t)p.rows_a * (uint64_t)p.lda * 2u));
  int rows = 0;
  auto a_off = [&](int i, int lim) {
    const int row = 16 * i + (lane >> 2);
    const int kc = (lane & 3) ^ ((row >> 1) & 3);
    uint32_t off = 0x80000000u;  // rows past the tile's routes read as zero
    if (row < lim) {
      const int rt = s_rt[row];
      const int src = MODE == 0 ? rt / p.topk : rt;
      off = ((uint32_t)src * (uint32_t)p.lda + (uint32_t)(kc * 8)) * 2u;
    }
    return off;
  };
  uint32_t a_voff0 = 0x80000000u, a_voff4 = 0x80000000u;  // set once the route list is in LDS

  // ---- weights: the lane's pieces of run (st, k-step): the low halves of rows 8 q .. 8 q + 7
  // of word r, paired, at byte 16 lane of the run, the high halves at 1024 + 16 lane; the DMA
  // puts them at the
  // same lane's place in LDS.  Scales (16 bytes: the word's 8 columns) and zeros (the word)
  // of the k-step's group likewise, by lanes 0..15 ----
  const uint32_t stream_bytes = (uint32_t)p.tiles * (uint32_t)KS * 2048u;
  const uint32_t w_run = (uint32_t)(wave_on ? st : 0) * (uint32_t)KS * 2048u;  // + 16 lane
  u32x4 wrs, srs, zrs;  // expert ex's stream copy, scales and zeros
  auto set_expert = [&](int ex) {
    wrs = rsrc_words((const char*)p.qw + (int64_t)ex * stream_bytes, wave_on ? stream_bytes : 0u);
    srs = rsrc_words(p.sc + (int64_t)ex * ngroups * p.N, (uint32_t)ngroups * (uint32_t)p.N * 2u);
    zrs = rsrc_words(ZP ? (const void*)(p.qz + (int64_t)ex * ngroups * NW) : (const void*)p.sc,
                     ZP ? (uint32_t)ngroups * (uint32_t)NW * 4u : 0u);
  };
  // DMA instructions per k-step: activation (1, or 2 for waves stl < A_TWO), weight (2),
  // scales (1), zeros (1)
  constexpr int NB_REST = 2 + 1 + (ZP ? 1 : 0);

  // piece `part` (0..3) of the request for this half's k-step s, into the slot at byte address
  // `slot` (slot s % PD; the k-loop keeps the slot indices as counters instead of dividing by
  // PD for every piece: T = 512 gate_up 64.0 -> 63.5 us, down 38.1 -> 37.8 us)
  // (ln: the lane index)
  auto issue_part = [&](int s, int part, int ln, uint32_t slot) __attribute__((always_inline)) {
    const int ks = s_first + s;
    if (part == 0) {
      const uint32_t abase = slot + (uint32_t)(A_OFF + kh * BM * CPR) * 16u;
      lds_dma16(ars, abase + (uint32_t)(stl * 64) * 16u, a_voff0, (uint32_t)(ks * BK * 2));
      if (stl < A_TWO) lds_dma16(ars, abase + (uint32_t)((kTST + stl) * 64) * 16u, a_voff4, (uint32_t)(ks * BK * 2));
    } else if (part == 1 || part == 2) {
      const int e2 = part - 1;
      lds_dma16(wrs, slot + (uint32_t)(W_OFF + (wave * 2 + e2) * 64) * 16u, w_run + (uint32_t)ln * 16u + (uint32_t)e2 * 1024u,
                (uint32_t)ks * 2048u);
    } else {
      const uint32_t g = (uint32_t)((ks * BK) >> lg);
      if (lane < 16) {  // one copy per word
        lds_dma16(srs, slot + (uint32_t)(S_OFF + wave * 16) * 16u, 16u * wc, g * (uint32_t)p.N * 2u);
        if constexpr (ZP)
          lds_dma4(zrs, slot + (uint32_t)Z_OFF * 16u + (uint32_t)(wave * 16) * 4u, 4u * wc, g * (uint32_t)NW * 4u);
      }
    }
  };
  // the first requests, one k-step at a time (weights, scales and zeros depend on the expert
  // only; activations on the route list)
  auto issue_wsz_s = [&](int s) {
    if (s < n_my)
#pragma unroll
      for (int part = 1; part < 4; ++part) issue_part(s, part, lane, lds0 + (uint32_t)s * SLOT_BYTES);
  };
  auto issue_a_s = [&](int s) {
    if (s < n_my) issue_part(s, 0, lane, lds0 + (uint32_t)s * SLOT_BYTES);
  };

  // ---- the row tile is found from the route counts (one round of loads).  Before that, the
  // block bets on the usual prefill case, every expert with 1 .. BM - 1 routes: row tile t is
  // then expert t's only tile, its routes from 0, min(count, BM) of them.  The counts, the bet
  // expert's count and first BM list entries (to LDS by DMA) and k-step 0's weights, scales and
  // zeros go out first; once the list has landed, k-step 0's activation rows, then k-steps
  // 1 .. PD - 2 whole, one after another.  So every block's first k-step is at the head of the
  // memory queues (the first requests of all blocks are a 31 MB burst; requested weights-first
  // for all four k-steps, k-step 0's activations came last; T = 512 A/Bs on two boxes: down
  // 36.2 -> 34.8 and 35.8 -> 35.1 us, gate_up 56.1 -> 55.2 and 55.9 -> 56.0 us), and the
  // k-loop's own waits (PD - 2 k-steps in flight) cover the
  // first k-step.  A lost bet waits for all of them and asks again, so the bet changes only
  // when the data arrive ----
  const bool bet = t_tile < E;  // block-uniform
  // fp32 route weights (read by the epilogue only) go to LDS by DMA, with k-step 0's requests
  const bool rw_dma = MODE == 0 && p.rw_dtype == AWQ_DTYPE_F32;
  auto route_weight_dma = [&](int rt) {
    const uint32_t sw_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) float*)&s_w[0];
    lds_dma4(rsrc_words(p.rw, (uint32_t)p.R * 4u), sw_lds + (uint32_t)wave * 256u, (uint32_t)rt * 4u, 0u);
  };
  // wave 0: the counts of experts 0..63 and the bet expert's count (assembly loads, waited for
  // below by count: the DMAs after them stay in flight)
  uint32_t cnt0 = 0, cnt_bet = 0;
  if (wave == 0) {
    const u32x4 crs = rsrc_words(p.counts, (uint32_t)E * 4u);  // lanes past E read zero
    asm volatile("buffer_load_dword %0, %1, %2, %3 offen" : "=v"(cnt0) : "v"((uint32_t)lane * 4u), "s"(crs), "s"(0u) : "memory");
    if (bet)
      asm volatile("buffer_load_dword %0, %1, %2, %3 offen" : "=v"(cnt_bet) : "v"((uint32_t)t_tile * 4u), "s"(crs), "s"(0u) : "memory");
  }
  int e_cur = bet ? t_tile : 0;
  if (bet && tid < BM) {  // waves 0 and 1: list entries 0 .. BM - 1 of expert e_cur into s_rt
    const uint32_t rt_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) int*)&s_rt[0];
    lds_dma4(rsrc_words(p.lists + (int64_t)e_cur * p.R, (uint32_t)p.R * 4u), rt_lds + (uint32_t)wave * 256u,
             (uint32_t)tid * 4u, 0u);
  }
  set_expert(e_cur);
  if (bet) {
    issue_wsz_s(0);
    // the list (and wave 0's counts) landed: k-step 0's NB_REST DMAs were issued after them
    if (wave < 2) {
      if (n_my >= 1) AWQ_WAIT_VMCNT(NB_REST);
      else AWQ_WAIT_VMCNT0();
    }
    if (wave == 0) {
      pin_after_wait(cnt_bet);
      if (lane == 0) s_tile[3] = min((int)cnt_bet, BM);
    }
    __syncthreads();
    const int lim = s_tile[3];  // the bet's routes (a won bet's tile has exactly these)
    a_voff0 = a_off(stl, lim);
    if (stl < A_TWO) a_voff4 = a_off(kTST + stl, lim);
    issue_a_s(0);
    if (rw_dma && tid < lim) route_weight_dma(s_rt[tid]);
    for (int s = 1; s < PD - 1; ++s) {
      issue_wsz_s(s);
      issue_a_s(s);
    }
  }
  if (wave == 0) {
    if (!bet) AWQ_WAIT_VMCNT0();
    pin_after_wait(cnt0);
    int te, tm0, trows;
    moe_row_tile_wave(p.counts, E, t_tile, te, tm0, trows, true, (int)cnt0);
    if (lane == 0) {
      s_tile[0] = te;
      s_tile[1] = tm0;
      s_tile[2] = trows;
    }
  }
  __syncthreads();
  const int e = __builtin_amdgcn_readfirstlane(s_tile[0]);
  const int m0 = __builtin_amdgcn_readfirstlane(s_tile[1]);
  rows = __builtin_amdgcn_readfirstlane(s_tile[2]);
  if (e < 0) {  // past the last row tile (whole block); no LDS DMA may land after the exit
    AWQ_WAIT_VMCNT0();
    return;
  }
  const int n_mt = (rows + 15) >> 4;  // token tiles holding routes (block-uniform)
  const bool won = bet && e == e_cur && m0 == 0;  // block-uniform
  if (won) {
    // s_rt holds the tile's routes and the first requests cover them; 16-bit route weights by
    // plain loads
    if (MODE == 0 && !rw_dma && tid < rows) s_w[tid] = load_route_weight(p.rw, p.rw_dtype, s_rt[tid]);
  } else {
    AWQ_WAIT_VMCNT0();  // this wave's bet DMAs (its slot, s_rt and s_w parts) have landed
    e_cur = e;
    set_expert(e);
    int rt = 0;
    if (tid < rows) {
      rt = p.lists[(int64_t)e * p.R + m0 + tid];
      s_rt[tid] = rt;
      if (MODE == 0 && !rw_dma) s_w[tid] = load_route_weight(p.rw, p.rw_dtype, rt);
    }
    __syncthreads();
    a_voff0 = a_off(stl, rows);
    if (stl < A_TWO) a_voff4 = a_off(kTST + stl, rows);
    for (int s = 0; s < PD - 1; ++s) {
      issue_wsz_s(s);
      issue_a_s(s);
      if (s == 0 && rw_dma && tid < rows) route_weight_dma(rt);
    }
  }

  // LDS byte offsets (within a slot) this lane reads
  auto a_rd = [&](int ln) __attribute__((always_inline)) {
    const int rr = ln & 15, qq = ln >> 4;
    return (uint32_t)(A_OFF + kh * BM * CPR + rr * CPR + (qq ^ ((rr >> 1) & 3))) * 16u;
  };
  auto w_rd = [&](int ln) __attribute__((always_inline)) { return (uint32_t)ln * 16u + (uint32_t)(W_OFF + wave * 128) * 16u; };
  auto s_rd = [&](int ln) __attribute__((always_inline)) { return (uint32_t)(ln & 15) * 16u + (uint32_t)(S_OFF + wave * 16) * 16u; };
  auto z_rd = [&](int ln) __attribute__((always_inline)) {
    return (uint32_t)(ln & 15) * 4u + (uint32_t)Z_OFF * 16u + (uint32_t)(wave * 16) * 4u;
  };
  auto lds16 = [](uint32_t addr) __attribute__((always_inline)) {
    return *(const __attribute__((address_space(3))) u32x4*)(uintptr_t)addr;
  };
  auto lds4 = [](uint32_t addr) __attribute__((always_inline)) {
    return *(const __attribute__((address_space(3))) uint32_t*)(uintptr_t)addr;
  };
  // byte address of k-step s's slot, opaque to the compiler (no per-slot copies of the lane
  // read addresses are kept)
  auto slot_of = [&](int cs) __attribute__((always_inline)) {  // cs: the slot index s % PD
    uint32_t b = lds0 + (uint32_t)cs * SLOT_BYTES;
    asm volatile("" : "+v"(b));
    return b;
  };

  const MagicK mk = magic_consts_s();
  // the exponent bytes of a nibble pair's biased zeros (0x6400 | z, 0x5400 | z << 4), in an
  // SGPR so that one byte permute can merge them with the zero word's byte
  uint32_t zmag = 0x54006400u;
  asm volatile("" : "+s"(zmag));
  const bool sb = scale_bf16 != 0;

  // the rest specialized on the number of token tiles holding routes (block-uniform)
  auto body = [&](auto nmt_c) __attribute__((always_inline)) {
    constexpr int NMT = decltype(nmt_c)::value;
    f32x4 acc[8][NMT];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int mt = 0; mt < NMT; ++mt) acc[i][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

    int cur_group = -1;
    // the group's constants.  fp16 (FAST): the raw scale words (column c in half c & 1 of word
    // c >> 1) and the biased zeros of each nibble pair in one register (nibble 2 j in the low
    // half, 2 j + 1 in the high half); each nibble's packed subtract and multiply read their
    // halves through operand selects, so no per-nibble constant is formed in the k-loop.  Six
    // token tiles (192 accumulator registers) hold the zero word instead and form each pair's
    // zeros before the pair (one byte permute and one AND), which keeps the k-loop within the
    // 256 registers of two waves per SIMD.  (Against per-nibble broadcast constants, and six
    // tiles forming each nibble's zero from opaque copies of the zero word and the lane
    // offsets anew per k-step: T = 512 gate_up 60.2 -> 55.5 us, down 37.8 -> 35.8 us,
    // kernel-trace A/B on one box, two alternating runs each.)
    constexpr bool PACK = FAST;
    constexpr bool ZWORD = PACK && NMT >= 6;
    ColConst cc[8];
    u32x4 s4p = {0u, 0u, 0u, 0u};
    uint32_t zmp[4] = {0u, 0u, 0u, 0u};
    uint32_t zwp = 0u;
    // byte j of the zero word into bytes 0 and 2, the exponent bytes into 1 and 3, masked to
    // the nibbles: the biased zeros of nibbles 2 j and 2 j + 1
    auto zero_pair = [&](uint32_t zw, int j) __attribute__((always_inline)) {
      return __builtin_amdgcn_perm(zmag, zw, 0x07000500u | ((uint32_t)j << 16) | (uint32_t)j) & 0xFFF0FF0Fu;
    };
    // one k-step from the slot at sb0; between nibble pairs, the pieces of request `req`
    // REQV: the request is known to exist (the main part of the k-loop)
    auto compute = [&](uint32_t sb0, int s, int req, uint32_t rslot, auto reqv) __attribute__((always_inline)) {
      constexpr bool REQV = decltype(reqv)::value;
      const int ln = lane;
      const int g = ((s_first + s) * BK) >> lg;
      if (g != cur_group) {  // wave-uniform
        WordSZ sz;
        sz.s4 = lds16(sb0 + s_rd(ln));
        sz.zw = ZP ? lds4(sb0 + z_rd(ln)) : 0x88888888u;
        if constexpr (PACK) {
          s4p = sz.s4;
          if constexpr (ZWORD) zwp = sz.zw;
          else
#pragma unroll
            for (int j = 0; j < 4; ++j) zmp[j] = zero_pair(sz.zw, j);
        } else {
          prep_consts<false, FAST>(sz, sb, cc);
        }
        cur_group = g;
      }
      u32x4 af[NMT];
#pragma unroll
      for (int mt = 0; mt < NMT; ++mt) af[mt] = lds16(sb0 + a_rd(ln) + (uint32_t)(mt * 16 * CPR * 16));
      const u32x4 wv0 = lds16(sb0 + w_rd(ln)), wv1 = lds16(sb0 + w_rd(ln) + 1024u);
      // the word at k-rows 8 q .. 8 q + 7, rows (2v, 2v + 1) paired into lo / hi 16-bit halves
      // by the packer (moe_pack_stream_kernel)
      uint32_t mlo[4], mhi[4];
      uint32_t zcur = 0u;  // ZWORD: the current nibble pair's biased zeros
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        mlo[v] = wv0[v];
        mhi[v] = wv1[v];
      }
      // nibble I's operand from the group's constants
      auto operand = [&](auto i_c) __attribute__((always_inline)) {
        constexpr int I = decltype(i_c)::value;
        if constexpr (PACK) {
          constexpr int c = nib_col<false>(I);
          if constexpr (ZWORD && (I & 1) == 0) zcur = zero_pair(zwp, I >> 1);
          const f16x2 zh = as_h2(ZWORD ? zcur : zmp[I >> 1]);
          const f16x2 zb = (I & 1) ? __builtin_shufflevector(zh, zh, 1, 1) : __builtin_shufflevector(zh, zh, 0, 0);
          const f16x2 sh = as_h2(s4p[c >> 1]);
          const f16x2 sc = (c & 1) ? __builtin_shufflevector(sh, sh, 1, 1) : __builtin_shufflevector(sh, sh, 0, 0);
          u32x4 b;
#pragma unroll
          for (int u = 0; u < 4; ++u) b[u] = as_u((as_h2(magic_bits<I & 3>(I < 4 ? mlo[u] : mhi[u], mk)) - zb) * sc);
          return b;
        } else {
          return rows_operand<I, FAST, T>(mlo, mhi, cc[I], mk);
        }
      };
#define AWQ_RB_NIB(I)                                                                       \
      {                                                                                     \
        const u32x4 b = operand(std::integral_constant<int, I>{});                          \
        _Pragma("unroll") for (int mt = 0; mt < NMT; ++mt)                                  \
          acc[I][mt] = MfmaOp<T>::run(af[mt], b, acc[I][mt]);                               \
      }
#define AWQ_RB_REQ(PART)                                                                    \
      if (REQV || req >= 0) {                                                               \
        __builtin_amdgcn_sched_barrier(0);                                                  \
        issue_part(req, PART, ln, rslot);                                                   \
        __builtin_amdgcn_sched_barrier(0);                                                  \
      }
      AWQ_RB_NIB(0) AWQ_RB_NIB(1) AWQ_RB_REQ(0)
      AWQ_RB_NIB(2) AWQ_RB_NIB(3) AWQ_RB_REQ(1)
      AWQ_RB_NIB(4) AWQ_RB_NIB(5) AWQ_RB_REQ(2)
      AWQ_RB_NIB(6) AWQ_RB_NIB(7) AWQ_RB_REQ(3)
#undef AWQ_RB_REQ
#undef AWQ_RB_NIB
    };

    // the requests for this half's k-steps 0 .. PD - 2 went out one k-step after another (with
    // the route list, counts and route weights before k-step 1's): the k-loop's waits below
    // cover them
    int cs = 0, rs = PD - 1;  // slot indices of k-step s and of request s + PD - 1
    int s = 0;
    // main part: k-steps whose request s + PD - 1 exists in both halves (n_my >= n0 - 1) and
    // with PD - 2 requests in flight after this k-step's, so the waits and the request need no
    // run-time choices (T = 512 gate_up 64.0 -> 62.1 us, down 38.2 -> 36.9 us against one loop
    // with those choices in every k-step); the last PD k-steps run the general form
    for (const int n_main = n0 - PD; s < n_main; ++s) {
      if (stl < A_TWO) AWQ_WAIT_VMCNT(3 * (NB_REST + 2));
      else AWQ_WAIT_VMCNT(3 * (NB_REST + 1));
      __syncthreads();
      compute(slot_of(cs), s, s + PD - 1, lds0 + (uint32_t)rs * SLOT_BYTES, std::true_type{});
      cs = cs == PD - 1 ? 0 : cs + 1;
      rs = rs == PD - 1 ? 0 : rs + 1;
    }
    for (; s < n0; ++s) {
      // this k-step's DMAs have landed (the PD - 2 after it may stay in flight)
      if (s < n_my) {
        const int ahead = min(n_my - 1 - s, PD - 2);  // wave-uniform
        static_assert(PD - 2 == 3, "the waits below cover three k-steps in flight");
        if (stl < A_TWO) {
          constexpr int NB = NB_REST + 2;
          if (ahead == 3) AWQ_WAIT_VMCNT(3 * NB);
          else if (ahead == 2) AWQ_WAIT_VMCNT(2 * NB);
          else if (ahead == 1) AWQ_WAIT_VMCNT(NB);
          else AWQ_WAIT_VMCNT0();
        } else {
          constexpr int NB = NB_REST + 1;
          if (ahead == 3) AWQ_WAIT_VMCNT(3 * NB);
          else if (ahead == 2) AWQ_WAIT_VMCNT(2 * NB);
          else if (ahead == 1) AWQ_WAIT_VMCNT(NB);
          else AWQ_WAIT_VMCNT0();
        }
      }
      // every wave's share of the k-step has landed, and slot (s + PD - 1) % PD, read in the
      // previous k-step, is free
      __syncthreads();
      if (s < n_my) compute(slot_of(cs), s, s + PD - 1 < n_my ? s + PD - 1 : -1, lds0 + (uint32_t)rs * SLOT_BYTES, std::false_type{});
      cs = cs == PD - 1 ? 0 : cs + 1;
      rs = rs == PD - 1 ? 0 : rs + 1;
    }

    // ---- the K-halves meet.  down (and bf16 gate_up, short of registers for the exchange
    // below): the second half's sums go through LDS to the first-half wave, which stores every
    // row.  fp16 gate_up (whose epilogue also evaluates the activation): both finish the tile, the first-half wave of a stream tile taking token tiles 0 .. H0 - 1
    // and the second-half wave the rest; each sends its partial sums of the other's tiles
    // (16 bytes per lane and value) and adds the partner's to its own (a two-term fp32 sum is
    // the same in either order).  Two rounds of four nibbles each ----
    constexpr bool SPLIT = MODE == 0 && FAST;
    constexpr int H0 = SPLIT ? (NMT + 1) / 2 : NMT;  // token tiles the first half finishes
    if constexpr (SPLIT) {
      f32x4* red4 = (f32x4*)&lds_all[0];  // [wave][4 nibbles][H0 tiles][64 lanes]
      static_assert(NWV * 4 * H0 * 64 * 16 <= PD * SLOT * 16, "the exchange fits the stage slots");
      const int partner = wave ^ kTST;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        __syncthreads();  // LDS free (stage reads done / previous round consumed)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int mt = 0; mt < NMT; ++mt) {
            if (kh == 0 ? mt >= H0 : mt < H0)  // the partner's tile (wave-uniform)
              red4[((wave * 4 + i) * H0 + (kh == 0 ? mt - H0 : mt)) * 64 + lane] = acc[4 * h + i][mt];
          }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int mt = 0; mt < NMT; ++mt) {
            if (kh == 0 ? mt < H0 : mt >= H0)  // this wave's tile
              acc[4 * h + i][mt] += red4[((partner * 4 + i) * H0 + (kh == 0 ? mt : mt - H0)) * 64 + lane];
          }
      }
    } else {
      constexpr int NVH = 4 * NMT * 4;  // floats per lane per round
      float* red = (float*)&lds_all[0];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        __syncthreads();  // LDS free (stage reads done / previous round consumed)
        if (kh == 1) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
              for (int v = 0; v < 4; ++v) red[((stl * NVH) + (i * NMT + mt) * 4 + v) * 64 + lane] = acc[4 * h + i][mt][v];
        }
        __syncthreads();
        if (kh == 0) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
              for (int v = 0; v < 4; ++v) acc[4 * h + i][mt][v] += red[((stl * NVH) + (i * NMT + mt) * 4 + v) * 64 + lane];
        }
      }
      if (kh == 1) return;
    }

    // ---- epilogue of this wave's token tiles: acc[I][mt][v] = row 16 mt + 4 q + v, column
    // 8 word + nib_col(I) ----
    auto epilogue = [&](auto kind_c) __attribute__((always_inline)) {
      constexpr int KIND = decltype(kind_c)::value;
      // the lane's first output column as a byte address and the row stride in bytes, so that a
      // row's address is one 32 x 32 -> 64-bit multiply-add of its route index (the host keeps
      // every per-route buffer, and so every route index and row stride, below 2^31 bytes)
      constexpr uint32_t EB = MODE == 0 ? 2u : 4u;  // bytes per output value
      const int ocol = MODE == 0 ? (r < 8 ? 8 * word : 8 * (word - p.half) + 4) : 8 * word;
      const uint64_t obase = (uint64_t)(uintptr_t)p.out + (uint64_t)(int64_t)ocol * EB;
      const uint32_t ostride = (uint32_t)p.ldo * EB;
#pragma unroll
      for (int mt = 0; mt < NMT; ++mt) {
        if (kh == 0 ? mt >= H0 : mt < H0) continue;  // the partner's tile (wave-uniform)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int m = 16 * mt + 4 * q + v;
          if constexpr (MODE == 0) {
            // lanes 0..7 hold gate sums, lanes 8..15 the up sums of the same columns.  Lane r < 8
            // finishes columns 0..3 of its word and lane r + 8 columns 4..7: per column pair, two
            // row rotations by 8 that each write one half of the row (DPP bank mask; the other
            // half keeps its own value) give every lane the gate and the up sum of its column.
            // Each source value is first taken into a register of its own (a DPP move fed
            // directly from an element of the accumulator tuple was compiled to read element 0).
            float gt[4], ut[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              float a = acc[col_nib<false>(j)][mt][v], b = acc[col_nib<false>(4 + j)][mt][v];
              asm volatile("" : "+v"(a), "+v"(b));
              gt[j] = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, a), __builtin_bit_cast(int, b), 0x128, 0xF, 0xC, false));
              ut[j] = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, b), __builtin_bit_cast(int, a), 0x128, 0xF, 0x3, false));
            }
            if (m < rows && word >= 0) {
              const int rt = s_rt[m];
              const float wgt = s_w[m];
              float h[4];
#pragma unroll
              for (int j = 0; j < 4; ++j) h[j] = gated_act_fast<KIND>(gt[j]) * ut[j] * wgt;
              *(u32x2*)(uintptr_t)(obase + (uint64_t)(uint32_t)rt * ostride) = u32x2{pack2<T>(h[0], h[1]), pack2<T>(h[2], h[3])};
            }
          } else {
            if (m < rows && word >= 0) {
              const int rt = s_rt[m];
              float y[8];
#pragma unroll
              for (int I = 0; I < 8; ++I) y[nib_col<false>(I)] = acc[I][mt][v];
              float* dst = (float*)(uintptr_t)(obase + (uint64_t)(uint32_t)rt * ostride);
              *(f32x4*)dst = f32x4{y[0], y[1], y[2], y[3]};
              *(f32x4*)(dst + 4) = f32x4{y[4], y[5], y[6], y[7]};
            }
          }
        }
      }
    };
    if (MODE == 0 && p.act_kind == 1) epilogue(std::integral_constant<int, 1>{});  // kernel-uniform
    else epilogue(std::integral_constant<int, 0>{});
  };
  switch (n_mt) {
    case 1: body(std::integral_constant<int, 1>{}); break;
    case 2: body(std::integral_constant<int, 2>{}); break;
    case 3: body(std::integral_constant<int, 3>{}); break;
    case 4: body(std::integral_constant<int, 4>{}); break;
    case 5: body(std::integral_constant<int, 5>{}); break;
    default: body(std::integral_constant<int, 6>{}); break;
  }
}

}  // namespace awq

namespace awq_host {

template <int MODE, bool ZP, typename T, bool FAST>
void launch_moe_tile_t(const awq::MoeArgs& a, int E, int sbf, hipStream_t st) {
  const int col_groups = (int)awq::cdiv(a.tiles, awq::kTST);
  // each expert adds at most one partial tile; rounded up to whole rounds of the 8 XCDs (row
  // tiles past the last one exit at once)
  const int64_t tiles_m = (awq::cdiv(a.R, awq::kTBM) + E + 7) / 8 * 8;
  hipLaunchKernelGGL((awq::moe_tile_kernel<MODE, ZP, T, FAST>), dim3((unsigned)(tiles_m * col_groups)),
                     dim3(128 * awq::kTST), 0, st, a, sbf, E, col_groups);
}

template <int MODE>
void launch_moe_tile_mode(const awq::MoeArgs& a, int E, bool zp, int act, int sbf, hipStream_t st) {
  using awq::bf16;
  using awq::f16;
  if (act == AWQ_DTYPE_BF16) {
    zp ? launch_moe_tile_t<MODE, true, bf16, false>(a, E, sbf, st) : launch_moe_tile_t<MODE, false, bf16, false>(a, E, sbf, st);
  } else if (!sbf) {
    zp ? launch_moe_tile_t<MODE, true, f16, true>(a, E, sbf, st) : launch_moe_tile_t<MODE, false, f16, true>(a, E, sbf, st);
  } else {
    zp ? launch_moe_tile_t<MODE, true, f16, false>(a, E, sbf, st) : launch_moe_tile_t<MODE, false, f16, false>(a, E, sbf, st);
  }
}

}  // namespace awq_host
