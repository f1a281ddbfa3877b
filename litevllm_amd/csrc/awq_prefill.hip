// Prefill GEMM (M > 32) on the stream layout of the weights (the copy the decode kernel also
// reads), gfx950: the role of _awq_native_tiled_gemm_autotuned
// (vllm/kernels/triton/awq_fused_gemm.py:2296-2392).
//
//  * Block tile 256 (M) x 64 NWN (N), k-stages of 64, 2 x NWN waves (two per SIMD at NWN = 4),
//    wave tile 128 x 64: 4 x 2 accumulators of v_mfma_f32_32x32x16_{f16,bf16}.
//  * Each k-stage the block dequantizes its weight tile once into LDS as [n][k] half values.
//    A thread takes one 16-byte piece of the stream layout: one packed word's four nibble
//    positions (low or high half) over 8 k-rows, already paired row by row, so the exact
//    magic-number dequant, (q - z) * s rounded once, needs no byte permutes, and each nibble
//    position gives one 16-byte chunk (8 k-values of one column).  That is about 60 VALU
//    instructions per thread and stage against 32 MFMAs per wave, and on this part VALU work
//    overlaps the matrix pipe only in part (its issue time adds to the MFMAs' almost in full),
//    so it is kept small: with groups of 128 rows or more the column constants (scale, biased
//    zero) and their loads come once per pair of stages.
//  * The activation tile goes straight from memory into LDS (buffer loads with the LDS
//    modifier) one stage ahead; the weight pieces, scales and zeros of stage s + 2 are
//    requested while stage s computes and wait in registers.
//  * LDS is double-buffered; one barrier per stage separates writing stage s + 1 from reading
//    stage s.  The stage loop is unrolled by two, so both buffers are addressed with immediate
//    offsets from loop-invariant lane addresses.
//  * 16-byte chunks are XOR-swizzled per row so that neither the operand reads (32 consecutive
//    rows at one chunk) nor the dequant stores (8 lanes, rows 8 apart) draw LDS bank conflicts.
//  * Blocks are dealt to the 8 XCDs so that each XCD works through contiguous tiles.
#include "awq_common.h"
#include "awq_launch.h"

namespace awq {

typedef float f32x16 __attribute__((ext_vector_type(16)));

template <typename T> struct Mfma32;
template <> struct Mfma32<f16> {
  static __device__ __forceinline__ f32x16 run(const u32x4& a, const u32x4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                  0);
  }
};
template <> struct Mfma32<bf16> {
  static __device__ __forceinline__ f32x16 run(const u32x4& a, const u32x4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  }
};

// 16-byte chunk swizzle of the 128-byte LDS rows (activation rows m, weight rows n): chunk kc of
// row r sits at slot kc ^ swz(r).  Measured with SQ_LDS_BANK_CONFLICT on gfx950: an operand read
// of 32 consecutive rows at one chunk is conflict-free with (r ^ r / 8) & 7 (r & 7 alone costs
// about 16 conflict cycles per read), and a store by 8 lanes is conflict-free when their slots
// differ, which (r ^ r / 8) & 7 gives the dequant stores (rows 8 apart).
__device__ __forceinline__ int ps_swz(int r) { return (r ^ (r >> 3)) & 7; }

constexpr int kPSBM = 256, kPSBK = 64;

template <int NWN, bool ZP, typename T, bool FAST, bool GPAIR>
__global__ void __launch_bounds__(128 * NWN, 2) prefill_stream_kernel(const GemmArgs p, int scale_bf16, int tiles_m,
                                                                      int tiles_n, int log2g, int n_off, int s_per) {
  constexpr int NT = 128 * NWN;                // threads
  constexpr int BM = kPSBM, BN = 64 * NWN, BK = kPSBK;
  constexpr int CPR = BK / 8;                  // 16-byte chunks per LDS row
  constexpr int ACH = BM * CPR / NT;           // activation chunks per thread per stage
  constexpr int BT = BN / 128;                 // stream tiles (128 columns) per block tile
  static_assert(BT * 2 * 2 * 64 == NT, "one 16-byte weight piece per thread per stage");
  // one LDS block: activation stages [2][BM][CPR], weight stages [2][BN][CPR]; after the k loop
  // the same bytes hold the output tile [BM][BN] fp16 (BM * BN * 2 <= its size)
  __shared__ u32x4 lds_all[2 * BM * CPR + 2 * BN * CPR];
  static_assert(BM * BN * 2 <= (int)sizeof(lds_all), "output tile fits the stage buffers");
  u32x4(&lds_a)[2][BM * CPR] = *reinterpret_cast<u32x4(*)[2][BM * CPR]>(&lds_all[0]);
  u32x4(&lds_b)[2][BN * CPR] = *reinterpret_cast<u32x4(*)[2][BN * CPR]>(&lds_all[2 * BM * CPR]);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / NWN, wn = wave % NWN;
  const int l32 = lane & 31, lh = lane >> 5;

  const int ntiles = tiles_m * tiles_n;
  int bid = blockIdx.x;
  if ((ntiles & 7) == 0) bid = (bid & 7) * (ntiles >> 3) + (bid >> 3);
  const int tm = bid / tiles_n, tn = bid - tm * tiles_n;
  const int m0 = tm * BM, n0 = n_off + tn * BN;  // the launch covers columns n_off ..

  const int KS = p.K >> 5;                     // 32-row k-steps of the stream layout
  const int nst = (p.K + BK - 1) / BK;
  // split-K (s_per > 0): grid row blockIdx.y takes stages s_beg .. s_end - 1 (s_per even, so the
  // stage pairs that share constants stay whole)
  const int split = blockIdx.y;
  const int s_beg = s_per > 0 ? split * s_per : 0;
  const int s_end = s_per > 0 ? min(s_beg + s_per, nst) : nst;
  const int ngroups = p.K / p.G;
  const int NW = p.N >> 3;

  // ---- the thread's weight piece: wave (t, ks, e), lane (q, r) ----
  const int pt = wave >> 2, pks = (wave >> 1) & 1, pe = wave & 1;
  const int pq = lane >> 4, pr = lane & 15;
  const int tg = (n0 >> 7) + pt;               // global stream tile
  const int word = tg * 16 + pr;
  const int wld = word < NW ? word : NW - 1;   // scales/zeros of columns past N: any valid word
  const int kchunk = 4 * pks + pq;             // the piece's k-chunk within a stage
  // piece offset of stage s: run (tg * KS + 2 s + pks), piece e, lane; s * 4096 rides in soffset
  const uint32_t w_voff = ((uint32_t)(tg * KS + pks) * 2048u) + (uint32_t)pe * 1024u + (uint32_t)lane * 16u;
  const uint32_t w_bytes = cdiv_u((uint32_t)NW, 16u) * 16u * (uint32_t)p.K * 4u;
  // LDS store address of each of the piece's 4 nibble positions (columns 8 r + col(4 e + P))
  uint32_t b_st[4];
#pragma unroll
  for (int P = 0; P < 4; ++P) {
    const int n = 128 * pt + 8 * pr + nib_col<false>(4 * pe + P);
    b_st[P] = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) u32x4*)&lds_b[0][n * CPR + (kchunk ^ ps_swz(n))];
  }

  // ---- activations: DMA instruction i of wave w fills chunks (w ACH + i) 64 + lane, i.e. row
  // 8 (w ACH + i) + lane / 8, slot lane % 8, holding k-chunk slot ^ swz(row) ----
  const uint64_t abase = (uint64_t)(uintptr_t)p.a;
  const u32x4 ars = {(uint32_t)abase, (uint32_t)(abase >> 32) & 0xFFFFu,
                     (uint32_t)((uint64_t)p.M * (uint64_t)p.lda * 2u), 0x00020000u};
  uint32_t a_voff[ACH];
  int a_kc[ACH];
#pragma unroll
  for (int i = 0; i < ACH; ++i) {
    const int row = 8 * (wave * ACH + i) + (lane >> 3);
    a_kc[i] = (lane & 7) ^ ps_swz(row);
    a_voff[i] = ((uint32_t)(m0 + row) * (uint32_t)p.lda + (uint32_t)(a_kc[i] * 8)) * 2u;
  }
  const uint32_t lds_a0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) u32x4*)&lds_a[0][wave * ACH * 64];
  const bool k_tail = (p.K % BK) != 0;

  // ---- operand read addresses: A rows 128 wm + 32 mt + lane % 32, B columns 64 wn + 32 nt +
  // lane % 32, k-chunk 2 j + lane / 32; swz of rows 32 apart differs by 4 when the row / 32 parity
  // differs, so one lane address per (j, parity) ----
  uint32_t ra[4][2], rb[4][2];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int kc = 2 * j + lh;
#pragma unroll
    for (int par = 0; par < 2; ++par) {
      const int row = 128 * wm + 32 * par + l32;
      ra[j][par] = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) u32x4*)&lds_a[0][row * CPR + (kc ^ ps_swz(row))];
      const int n = 64 * wn + 32 * par + l32;
      rb[j][par] = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) u32x4*)&lds_b[0][n * CPR + (kc ^ ps_swz(n))];
    }
  }

  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const MagicK mk = magic_consts();
  // weight pieces, scales and zero words of two stages in flight, slot = stage parity
  u32x4 bq[2];
  WordSZ bs[2];
  const uint64_t wbase = (uint64_t)(uintptr_t)p.qw;
  const u32x4 wrs = {(uint32_t)wbase, (uint32_t)(wbase >> 32) & 0xFFFFu, w_bytes, 0x00020000u};
  const u32x4 wrs0 = {(uint32_t)wbase, (uint32_t)(wbase >> 32) & 0xFFFFu, 0u, 0x00020000u};  // reads zero
  const uint64_t sbase = (uint64_t)(uintptr_t)p.sc, zbase = (uint64_t)(uintptr_t)(ZP ? (const void*)p.qz : (const void*)p.sc);
  const u32x4 srs = {(uint32_t)sbase, (uint32_t)(sbase >> 32) & 0xFFFFu, (uint32_t)((uint64_t)ngroups * p.N * 2u),
                     0x00020000u};
  const u32x4 zrs = {(uint32_t)zbase, (uint32_t)(zbase >> 32) & 0xFFFFu, (uint32_t)((uint64_t)ngroups * NW * 4u),
                     0x00020000u};
  constexpr int NB = ZP ? 3 : 2;  // loads of one stage's weight data
  // GPAIR (G >= 128): stages 2j and 2j + 1 lie in one group, so an odd stage loads its weight
  // piece only and reuses the column constants of the even stage before it (M = 2048,
  // N = 24576: 357.9 -> 350.6 us, bitwise equal, A/B on one box)
  constexpr int NB_ODD = GPAIR ? 1 : NB;
  ColConst cc[4];  // the column constants of the stage dequantized last (GPAIR; bf16)
  // fp16 (FAST): the group's constants two nibble positions per register, read through operand
  // selects: zmp[j] the biased zeros of positions 2 j and 2 j + 1 (0x6400 | z low, 0x5400 |
  // z << 4 high), sc2[j] their scales; one byte permute each (and one AND for the zeros) per
  // pair instead of a nibble extraction and a broadcast per position (M = 2048, N = 24576:
  // 345.3 -> 343.3 us, bitwise equal, A/B on one box)
  uint32_t zmp[2] = {0u, 0u}, sc2[2] = {0u, 0u};
  uint32_t zmag = 0x54006400u;  // the exponent bytes of the biased zeros, in an SGPR
  asm volatile("" : "+s"(zmag));
  const uint32_t ssel = pe ? 0x07060302u : 0x05040100u;  // half pe of two scale words

  auto dma_a = [&](int s, int buf) {
    const uint32_t dst = lds_a0 + (uint32_t)buf * (uint32_t)sizeof(lds_a[0]);
    if (k_tail && s * BK + BK > p.K) {  // wave-uniform: a last half stage's upper chunks read zero
#pragma unroll
      for (int i = 0; i < ACH; ++i)
        lds_dma16(ars, dst + (uint32_t)(i * 1024), s * BK + a_kc[i] * 8 >= p.K ? 0x80000000u : a_voff[i],
                  (uint32_t)(s * BK * 2));
    } else {
#pragma unroll
      for (int i = 0; i < ACH; ++i) lds_dma16(ars, dst + (uint32_t)(i * 1024), a_voff[i], (uint32_t)(s * BK * 2));
    }
  };
  // stage s's weight piece, scales and zero word into slot s & 1 (NB loads).  The stage's run
  // offset s * 4096 rides in soffset, which the buffer range check does not cover, so a piece
  // whose k-step 2 s + pks lies past K (stages past the last one, and the upper half of a last
  // half stage when K % 64 == 32) reads through an empty descriptor instead: zeros, no traffic.
  // Its activations are zero, so the zero piece adds nothing.
  auto load_b = [&](int s, int slot) {
    bq[slot] = asm_load16(2 * s + pks < KS && s < s_end ? wrs : wrs0, w_voff, (uint32_t)s * 4096u);
    if (GPAIR && slot == 1) return;  // odd stage (slot = stage parity): constants reused
    const int gi = min((s * BK + 8 * kchunk) >> log2g, ngroups - 1);
    bs[slot].s4 = asm_load16(srs, (uint32_t)((gi * p.N + 8 * wld) * 2), 0u);
    if constexpr (ZP) bs[slot].zw = asm_load4(zrs, (uint32_t)((gi * NW + wld) * 4));
    else bs[slot].zw = 0x88888888u;
  };
  // nibble position P of the piece -> the 16-byte chunk of its column (column 2 P + e of the
  // word: scale half e of scale word P, zero nibble 4 e + P), stored into buffer buf
  auto col_const = [&](int P, const WordSZ& bsz) {
    const uint32_t zn = (bsz.zw >> (16 * pe + 4 * P)) & 0xFu;
    const uint32_t sbits = (bsz.s4[P] >> (16 * pe)) & 0xFFFFu;
    ColConst c_;
    c_.zm = zero_magic(P & 1, zn);
    if constexpr (FAST) {
      c_.sc = sbits * 0x00010001u;
      c_.scf = 0.0f;
    } else {
      c_.sc = 0;
      c_.scf = scale_bf16 ? bf_bits2f((uint16_t)sbits) : h_bits2f((uint16_t)sbits);
    }
    return c_;
  };
  // fresh: the stage starts a group (its constants were loaded with it); otherwise (GPAIR, odd
  // stages) the previous stage's constants
  auto write_b = [&](int buf, int P, const u32x4& braw, const WordSZ& bsz, bool fresh) {
    f16x2 zz, ss;
    ColConst c_;
    if constexpr (FAST) {
      if ((!GPAIR || fresh) && (P & 1) == 0) {
        const uint32_t zb = (uint32_t)(2 * pe + (P >> 1));  // the zero word's byte of positions P, P + 1
        zmp[P >> 1] = __builtin_amdgcn_perm(zmag, bsz.zw, 0x07000500u | (zb << 16) | zb) & 0xFFF0FF0Fu;
        sc2[P >> 1] = __builtin_amdgcn_perm(bsz.s4[P + 1], bsz.s4[P], ssel);
      }
      const f16x2 zh = as_h2(zmp[P >> 1]), sh = as_h2(sc2[P >> 1]);
      zz = (P & 1) ? __builtin_shufflevector(zh, zh, 1, 1) : __builtin_shufflevector(zh, zh, 0, 0);
      ss = (P & 1) ? __builtin_shufflevector(sh, sh, 1, 1) : __builtin_shufflevector(sh, sh, 0, 0);
    } else {
      if (!GPAIR || fresh) cc[P] = col_const(P, bsz);
      c_ = cc[P];
    }
    u32x4 v;
#define AWQ_PS_CASE(PP)                                                                            \
    case PP: {                                                                                     \
      _Pragma("unroll") for (int u = 0; u < 4; ++u) {                                              \
        if constexpr (FAST) v[u] = as_u((as_h2(magic_bits<PP>(braw[u], mk)) - zz) * ss);           \
        else v[u] = deq2<FAST, T>(magic_bits<PP>(braw[u], mk), c_);                                \
      }                                                                                            \
      break;                                                                                       \
    }
    switch (P) {
      AWQ_PS_CASE(0) AWQ_PS_CASE(1) AWQ_PS_CASE(2)
      default: AWQ_PS_CASE(3)
    }
#undef AWQ_PS_CASE
    *(__attribute__((address_space(3))) u32x4*)(uintptr_t)(b_st[P] + (uint32_t)buf * (uint32_t)sizeof(lds_b[0])) = v;
  };
  auto rd = [&](uint32_t addr) { return *(__attribute__((address_space(3))) const u32x4*)(uintptr_t)addr; };
  // one 64-k stage from buffer cb; stage s + 1's weights (slot wslot) go to buffer cb ^ 1 --
  // after waiting (mid-stage) for their loads, issued one stage earlier: at most `pending` loads
  // issued after them may still be outstanding
  auto stage = [&](int cb, int wslot, bool dma_issued) {
    const int wb = cb ^ 1;
    const uint32_t ao = (uint32_t)cb * (uint32_t)sizeof(lds_a[0]), bo = (uint32_t)cb * (uint32_t)sizeof(lds_b[0]);
    u32x4 af[2][4], bf[2][2];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) af[0][mt] = rd(ra[0][mt & 1] + ao + (uint32_t)((mt >> 1) * 64 * CPR * 16));
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) bf[0][nt] = rd(rb[0][nt] + bo);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (j + 1 < 4) {
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
          af[(j + 1) & 1][mt] = rd(ra[j + 1][mt & 1] + ao + (uint32_t)((mt >> 1) * 64 * CPR * 16));
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) bf[(j + 1) & 1][nt] = rd(rb[j + 1][nt] + bo);
      }
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) acc[mt][nt] = Mfma32<T>::run(af[j & 1][mt], bf[j & 1][nt], acc[mt][nt]);
      if (j == 0) {
        // stage s + 1's weight loads (issued during stage s - 1) must have landed; the DMA and
        // the weight loads issued this stage may stay outstanding
        if (GPAIR && cb == 1) {  // this step's load_b was an odd stage's (weights only)
          if (dma_issued) AWQ_WAIT_VMCNT(ACH + NB_ODD);
          else AWQ_WAIT_VMCNT(NB_ODD);
        } else {
          if (dma_issued) AWQ_WAIT_VMCNT(ACH + NB);
          else AWQ_WAIT_VMCNT(NB);
        }
        pin_after_wait(bq[wslot]);
        pin_after_wait(bs[wslot].s4);
        pin_after_wait(bs[wslot].zw);
      }
      write_b(wb, j, bq[wslot], bs[wslot], wslot == 0);
      // issue order within the sub-step: the next sub-step's 6 operand reads spread over the
      // first 6 MFMAs, the dequant arithmetic in the gaps, its store last.  The sub-step runs at
      // raised wave priority, so the SIMD's other wave does not take issue slots between its
      // MFMAs (M = 2048, N = 24576: 349.4 -> 345.8 us, A/B on one box)
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                          // MFMA
        if (j + 1 < 4 && i < 6) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
        __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);                          // VALU
      }
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);                            // LDS write
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(0);
    }
  };

  // prologue: stage s_beg's activations and weights, the next stage's weights in flight
  dma_a(s_beg, 0);
  load_b(s_beg, 0);
  load_b(s_beg + 1, 1);
  AWQ_WAIT_VMCNT(NB_ODD);
  pin_after_wait(bq[0]);
  pin_after_wait(bs[0].s4);
  pin_after_wait(bs[0].zw);
#pragma unroll
  for (int P = 0; P < 4; ++P) write_b(0, P, bq[0], bs[0], true);
  __syncthreads();

  // stage s (buffer s & 1): request stage s + 1's activations and stage s + 2's weights (slot
  // s & 1), compute stage s and write stage s + 1's weights (slot (s + 1) & 1); one barrier per
  // stage once this wave's activation DMA has landed
  auto step = [&](int s, int cb) {
    const bool dma = s + 1 < s_end;
    if (dma) dma_a(s + 1, cb ^ 1);
    load_b(s + 2, cb);
    stage(cb, cb ^ 1, dma);
    if (GPAIR && cb == 1) AWQ_WAIT_VMCNT(NB_ODD);
    else AWQ_WAIT_VMCNT(NB);
    __syncthreads();
  };
  int s = s_beg;
  for (; s + 1 < s_end; s += 2) {
    step(s, 0);
    step(s + 1, 1);
  }
  if (s < s_end) step(s, 0);
  // the last stages' (empty) weight loads: their registers stay reserved until they have landed
  AWQ_WAIT_VMCNT0();
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    pin_after_wait(bq[k]);
    pin_after_wait(bs[k].s4);
    pin_after_wait(bs[k].zw);
  }

  if (s_per > 0) {
    // split-K: this range's fp32 sums (no bias) into partial[split]; 32 lanes store 32
    // consecutive columns of a row
    float* part = p.partial + (size_t)split * (size_t)p.M * (size_t)p.N;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int gcol = n0 + 64 * wn + 32 * nt + l32;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int grow = m0 + 128 * wm + 32 * mt + 8 * (r >> 2) + 4 * lh + (r & 3);
          if (grow < p.M && gcol < p.N) part[(size_t)grow * (size_t)p.N + gcol] = acc[mt][nt][r];
        }
    }
    return;
  }
  // Epilogue through LDS (the k loop's last barrier has passed, so every stage buffer is free):
  // lane l holds acc[mt][nt][r] = C[128 wm + 32 mt + 8 (r / 4) + 4 (l / 32) + r % 4]
  // [64 wn + 32 nt + l % 32] of the tile; each value (+ bias, rounded once) goes to the
  // row-major fp16 tile in LDS, whose 16-byte chunks are XOR-swizzled by row, and the block then
  // writes whole rows with 16-byte stores (instead of 2-byte stores scattered over 2 rows each).
  constexpr int CCH = BN / 8;  // 16-byte chunks per output row
  auto c_chunk = [&](int row, int ch) { return ch ^ (row & 15 & (CCH - 1)); };
  __attribute__((address_space(3))) uint16_t* cl = (__attribute__((address_space(3))) uint16_t*)(uintptr_t)(uint32_t)(
      uintptr_t)(__attribute__((address_space(3))) u32x4*)&lds_all[0];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int cc = 64 * wn + 32 * nt + l32;  // tile column
    const int colg = n0 + cc;
    const float bv = (p.bias && colg < p.N) ? load_bias(p.bias, p.bias_dtype, colg) : 0.0f;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = 128 * wm + 32 * mt + 8 * (r >> 2) + 4 * lh + (r & 3);
        cl[row * BN + c_chunk(row, cc >> 3) * 8 + (cc & 7)] = to_bits<T>(acc[mt][nt][r] + bv);
      }
    }
  }
  __syncthreads();
  constexpr int CHUNKS = BM * CCH;
  static_assert(CHUNKS % NT == 0, "");
#pragma unroll
  for (int j = 0; j < CHUNKS / NT; ++j) {
    const int i = j * NT + tid;
    const int row = i / CCH, ch = i % CCH;
    const int grow = m0 + row, gcol = n0 + 8 * ch;
    const u32x4 v = lds_all[row * CCH + c_chunk(row, ch)];
    if (grow < p.M && gcol < p.N) *(u32x4*)(p.c + (int64_t)grow * p.ldc + gcol) = v;
  }
}

// c[m][n .. n + 3] = round(sum over splits, in split order, of partial[s][m][n ..] + bias)
template <typename T>
__global__ void __launch_bounds__(256) prefill_split_reduce(const GemmArgs p, int S) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // 4-column group
  const int64_t n4 = p.N >> 2;
  if (i >= (int64_t)p.M * n4) return;
  const int64_t m = i / n4, n = (i - m * n4) * 4;
  const size_t plane = (size_t)p.M * (size_t)p.N;
  const float* src = p.partial + (size_t)m * (size_t)p.N + (size_t)n;
  f32x4 acc = *(const f32x4*)src;
  for (int s = 1; s < S; ++s) acc += *(const f32x4*)(src + (size_t)s * plane);
  float v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = acc[j] + (p.bias ? load_bias(p.bias, p.bias_dtype, (int)n + j) : 0.0f);
  *(u32x2*)(p.c + m * p.ldc + n) = u32x2{pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3])};
}

}  // namespace awq

namespace awq_host {
using namespace awq;

template <bool ZP, typename T, bool FAST>
static void launch_ps(const GemmArgs& a, int sbf, int log2g, hipStream_t st) {
  const int tm = (int)cdiv(a.M, kPSBM);
  const int tn4 = (int)cdiv(a.N, 256);
  const int cus = num_cus();
  // groups of 128 rows or more: both stages of a pair share their group
  const bool gpair = a.G >= 128;
  if (a.ksplit > 1) {
    // split-K: 256-column blocks over K ranges of whole stage pairs, then the ordered sum
    const int nst = (int)cdiv(a.K, kPSBK);
    const int per = (int)((cdiv(nst, a.ksplit) + 1) / 2 * 2);
    const int S = (int)cdiv(nst, per);
    const dim3 grid((unsigned)(tm * tn4), (unsigned)S);
    if (gpair) hipLaunchKernelGGL((prefill_stream_kernel<4, ZP, T, FAST, true>), grid, dim3(512), 0, st, a, sbf, tm, tn4, log2g, 0, per);
    else hipLaunchKernelGGL((prefill_stream_kernel<4, ZP, T, FAST, false>), grid, dim3(512), 0, st, a, sbf, tm, tn4, log2g, 0, per);
    const int64_t groups = (int64_t)a.M * (a.N / 4);
    hipLaunchKernelGGL((prefill_split_reduce<T>), dim3((unsigned)cdiv(groups, 256)), dim3(256), 0, st, a, S);
    return;
  }
  auto wide = [&](int tiles_n, int n_off) {
    if (gpair) hipLaunchKernelGGL((prefill_stream_kernel<4, ZP, T, FAST, true>), dim3(tm * tiles_n), dim3(512), 0, st, a, sbf, tm, tiles_n,
                       log2g, n_off, 0);
    else hipLaunchKernelGGL((prefill_stream_kernel<4, ZP, T, FAST, false>), dim3(tm * tiles_n), dim3(512), 0, st, a, sbf, tm, tiles_n,
                       log2g, n_off, 0);
  };
  auto narrow = [&](int tiles_n, int n_off) {
    if (gpair) hipLaunchKernelGGL((prefill_stream_kernel<2, ZP, T, FAST, true>), dim3(tm * tiles_n), dim3(256), 0, st, a, sbf, tm, tiles_n,
                       log2g, n_off, 0);
    else hipLaunchKernelGGL((prefill_stream_kernel<2, ZP, T, FAST, false>), dim3(tm * tiles_n), dim3(256), 0, st, a, sbf, tm, tiles_n,
                       log2g, n_off, 0);
  };
  // 256-column blocks (two waves per SIMD) once they cover three quarters of the CUs; below
  // that, twice as many 128-column blocks.  Measured on MI355X (K = 4096): M = 512, N = 24576
  // (192 blocks of 256 columns) 101 us against 134 us in 384 blocks of 128; M = 512, N = 12288
  // (96 blocks of 256 columns) 92 us against 74 us in 192 blocks of 128.
  if ((int64_t)tm * tn4 * 4 < (int64_t)cus * 3) {
    narrow((int)cdiv(a.N, 128), 0);
    return;
  }
  // Whole rounds of 256-column blocks, then a part round of them as 128-column blocks in a
  // second launch, where those fill the chip once: the part round runs at twice the blocks
  // for half the work each instead of leaving CUs idle (M = 2048, N = 12288: 384 blocks, 1.5
  // rounds).
  if (cus % tm == 0) {
    const int per_round = cus / tm;  // 256-column tiles per round of blocks
    const int full = tn4 / per_round * per_round;
    const int rest = (int)cdiv(a.N - full * 256, 128);
    if (full > 0 && rest > 0 && (int64_t)tm * rest <= cus) {
      wide(full, 0);
      narrow(rest, full * 256);
      return;
    }
  }
  wide(tn4, 0);
}

bool launch_prefill_stream(const GemmArgs& a, bool zp, int act, int sdt, hipStream_t st) {
  // group sizes that are powers of two (the kernel shifts by log2 G)
  if (a.G <= 0 || (a.G & (a.G - 1)) != 0) return false;
  const int log2g = __builtin_ctz((unsigned)a.G);
  const int sbf = (sdt == AWQ_DTYPE_BF16) ? 1 : 0;
  if (act == AWQ_DTYPE_F16) {
    if (sdt == AWQ_DTYPE_F16) zp ? launch_ps<true, f16, true>(a, sbf, log2g, st) : launch_ps<false, f16, true>(a, sbf, log2g, st);
    else zp ? launch_ps<true, f16, false>(a, sbf, log2g, st) : launch_ps<false, f16, false>(a, sbf, log2g, st);
  } else {
    zp ? launch_ps<true, bf16, false>(a, sbf, log2g, st) : launch_ps<false, bf16, false>(a, sbf, log2g, st);
  }
  return true;
}

}  // namespace awq_host
