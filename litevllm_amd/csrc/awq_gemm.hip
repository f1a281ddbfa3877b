// Prefill GEMM (M > 32) for the KN layouts (qweight [K, N/8]) on gfx950: the role of
// _awq_native_tiled_gemm_autotuned (vllm/kernels/triton/awq_fused_gemm.py:2296-2392).
//
//  * Block tile 256 (M) x 64 NWN (N), k-stages of 64, 2 x NWN waves, wave tile 128 x 64:
//    8 x 4 accumulators of v_mfma_f32_16x16x32_{f16,bf16} per wave.  NWN = 4 (256 columns,
//    one 512-thread block per CU) halves the activation traffic per flop of NWN = 2.
//  * Each k-stage the block dequantizes its weight tile once (every thread one packed word
//    over 4 k-rows, exact (q - z) * s) into LDS as [n][k] half values, so every wave reads
//    both MFMA operands with 16-byte LDS loads and no weight is dequantized twice in a block.
//  * The activation tile goes straight from memory to LDS (buffer loads with the LDS
//    modifier), one stage ahead; the packed weights, scales and zeros of stage s + 2 are
//    requested while stage s computes and wait in registers, so every global load has a
//    whole stage of MFMAs to arrive in.
//  * LDS is double-buffered: one barrier per stage separates writing stage s + 1 from
//    reading stage s.
//  * 16-byte LDS chunks are XOR-swizzled by row so that operand reads and the dequant writes
//    spread over the banks.
//  * Blocks are dealt to the 8 XCDs so that each XCD works through contiguous tiles (the same
//    activation row tile stays in its L2).
#include "awq_common.h"
#include "awq_launch.h"

namespace awq {

template <bool ZP>
__device__ __forceinline__ WordSZ load_sz(const GemmArgs& p, int g, int word) {
  WordSZ r;
  r.s4 = *(const u32x4*)(p.sc + (int64_t)g * p.N + 8 * word);
  r.zw = ZP ? p.qz[(int64_t)g * (p.N >> 3) + word] : 0x88888888u;
  return r;
}


// 16-byte chunk swizzles of 128-byte LDS rows (eight chunks).  Operand reads take 16
// consecutive rows; activation rows are stored whole, weight rows n = 8 w + c by lanes of
// neighbouring words w.  swz_a depends on the row's low bits only, so the A fragments of a
// wave sit at constant offsets from one lane address; swz_b also mixes in the word index so
// the dequant stores spread over the banks.
__device__ __forceinline__ int swz_a(int row) { return row & 7; }
__device__ __forceinline__ int swz_b(int n) { return (n ^ (n >> 4)) & 7; }

constexpr int kPBM = 256, kPBK = 64;

template <int NWN, bool SEQ, bool ZP, typename T, bool FAST>
__global__ void __launch_bounds__(128 * NWN, 2) prefill_kn_kernel(const GemmArgs p, int scale_bf16, int tiles_m,
                                                                  int tiles_n) {
  constexpr int NT = 128 * NWN;  // threads
  constexpr int BM = kPBM, BN = 64 * NWN, BK = kPBK;
  constexpr int WM = 128, WN = 64;
  constexpr int MTL = WM / 16, NTL = WN / 16;
  constexpr int CPR = BK / 8;            // 16-byte chunks per LDS row
  constexpr int ACH = BM * CPR / NT;     // activation chunks per thread per stage
  constexpr int BW = BN / 8;             // packed words per row of the tile
  static_assert(BW * (BK / 4) == NT, "one packed word x 4 k-rows per thread");
  // one LDS block: activation stages [2][BM][CPR], weight stages [2][BN][CPR]; after the k loop
  // the same bytes hold the output tile [BM][BN] fp16
  __shared__ u32x4 lds_all[2 * BM * CPR + 2 * BN * CPR];
  static_assert(BM * BN * 2 <= (int)sizeof(lds_all), "output tile fits the stage buffers");
  u32x4(&lds_a)[2][BM * CPR] = *reinterpret_cast<u32x4(*)[2][BM * CPR]>(&lds_all[0]);
  u32x4(&lds_b)[2][BN * CPR] = *reinterpret_cast<u32x4(*)[2][BN * CPR]>(&lds_all[2 * BM * CPR]);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform by construction
  const int q = lane >> 4, r = lane & 15;
  const int wave_m = wave / NWN, wave_n = wave % NWN;

  // XCD-aware tile order: blocks are dealt round-robin to the 8 XCDs; give each XCD a
  // contiguous range of tiles (row-tile major) so blocks sharing an activation row tile
  // share an L2.
  const int ntiles = tiles_m * tiles_n;
  int bid = blockIdx.x;
  if ((ntiles & 7) == 0) bid = (bid & 7) * (ntiles >> 3) + (bid >> 3);
  const int tm = bid / tiles_n, tn = bid - tm * tiles_n;
  const int m0 = tm * BM, n0 = tn * BN;

  const int NW = p.N >> 3;
  // dequant assignment: packed word bw of the tile, k-rows 4 kq .. 4 kq + 3 of the stage
  // (neighbouring lanes take neighbouring words: full 128-byte global row segments)
  const int bw = tid % BW, kq = tid / BW;
  const int bword = (n0 >> 3) + bw;
  const int bwld = bword < NW ? bword : NW - 1;  // columns past N are computed, never stored

  f32x4 acc[MTL][NTL];
#pragma unroll
  for (int mt = 0; mt < MTL; ++mt)
#pragma unroll
    for (int nt = 0; nt < NTL; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // K % 64 may be 32 (group size 32): the last stage's upper half reads zero activations
  const int nst = (p.K + BK - 1) / BK;
  const int ngroups = p.K / p.G;
  const MagicK mk = magic_consts();

  // activations: DMA instruction i of wave w fills 16-byte chunks c = (w ACH + i) 64 + lane of
  // the stage buffer, i.e. row c / 8, slot c % 8, which holds global chunk slot ^ swz_a(row);
  // rows past M read as zero (the descriptor's range check)
  const uint64_t abase = (uint64_t)(uintptr_t)p.a;
  const u32x4 ars = {(uint32_t)abase, (uint32_t)(abase >> 32) & 0xFFFFu,
                     (uint32_t)((uint64_t)p.M * (uint64_t)p.lda * 2u), 0x00020000u};  // raw, bounds-checked
  uint32_t a_voff[ACH];
  int a_k[ACH];  // the chunk's first k within a stage
#pragma unroll
  for (int i = 0; i < ACH; ++i) {
    const int c = (wave * ACH + i) * 64 + lane;
    const int row = c / CPR, ch = (c % CPR) ^ swz_a(row);
    a_k[i] = ch * 8;
    a_voff[i] = ((uint32_t)(m0 + row) * (uint32_t)p.lda + (uint32_t)(ch * 8)) * 2u;
  }
  const uint32_t lds_a0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) u32x4*)&lds_a[0][wave * ACH * 64];
  auto dma_a = [&](int s, int buf) {
    const bool tail = s * BK + BK > p.K;  // wave-uniform: only a last half stage checks columns
#pragma unroll
    for (int i = 0; i < ACH; ++i)
      lds_dma16(ars, lds_a0 + (uint32_t)buf * (uint32_t)sizeof(lds_a[0]) + (uint32_t)(i * 64 * 16),
                tail && s * BK + a_k[i] >= p.K ? 0x80000000u : a_voff[i], (uint32_t)(s * BK * 2));
  };
  // packed weights: the row offset of the stage rides in the SGPR offset; stages past the
  // last one go through an empty descriptor, and a last half stage checks its rows
  const uint32_t w_bytes = (uint32_t)((uint64_t)p.K * (uint64_t)NW * 4u);
  const uint32_t b_voff = ((uint32_t)(4 * kq) * (uint32_t)NW + (uint32_t)bwld) * 4u;
  uint32_t braw[4], bnext[4];
  WordSZ bsz, bsznext;
  auto load_b = [&](int s) {
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(p.qw, s < nst ? w_bytes : 0u);
    const bool tail = s * BK + BK > p.K;
    const uint32_t soff = (uint32_t)(s * BK) * (uint32_t)NW * 4u;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t vo = b_voff + (uint32_t)j * (uint32_t)NW * 4u;
      bnext[j] = __builtin_amdgcn_raw_buffer_load_b32(
          wrs, tail ? (int)(vo + soff) : (int)vo, tail ? 0 : (int)soff, 0);
    }
    bsznext = load_sz<ZP>(p, min((s * BK + 4 * kq) / p.G, ngroups - 1), bwld);
  };
  // nibble I of the thread's word over its 4 k-rows -> 8 bytes of LDS row n = 8 bw + col(I);
  // the nibble's constants are derived right here so only the raw group words stay live
  auto write_b_nib = [&](int buf, int I, const uint32_t (&lo)[2], const uint32_t (&hi)[2]) {
    u32x2 v;
    const bool sb = scale_bf16 != 0;
#define AWQ_PF_CASE(II, SRC, P)                                            \
    case II: {                                                             \
      const ColConst c_ = prep_const<II, SEQ, FAST>(bsz, sb);              \
      v[0] = deq2<FAST, T>(magic_bits<P>(SRC[0], mk), c_);                 \
      v[1] = deq2<FAST, T>(magic_bits<P>(SRC[1], mk), c_);                 \
      break;                                                               \
    }
    switch (I) {  // I is a constant after unrolling
      AWQ_PF_CASE(0, lo, 0) AWQ_PF_CASE(1, lo, 1) AWQ_PF_CASE(2, lo, 2) AWQ_PF_CASE(3, lo, 3)
      AWQ_PF_CASE(4, hi, 0) AWQ_PF_CASE(5, hi, 1) AWQ_PF_CASE(6, hi, 2)
      default: AWQ_PF_CASE(7, hi, 3)
    }
#undef AWQ_PF_CASE
    const int n = 8 * bw + nib_col<SEQ>(I);
    ((u32x2*)lds_b[buf])[(n * CPR + ((kq >> 1) ^ swz_b(n))) * 2 + (kq & 1)] = v;
  };
  auto mfma_sub = [&](int cb, int sub, int mt, const u32x4 (&bf)[NTL], const u32x4& af) {
    (void)cb; (void)sub;
#pragma unroll
    for (int nt = 0; nt < NTL; ++nt) acc[mt][nt] = MfmaOp<T>::run(af, bf[nt], acc[mt][nt]);
  };
  auto read_b = [&](int cb, int sub, u32x4 (&bf)[NTL]) {
#pragma unroll
    for (int nt = 0; nt < NTL; ++nt) {
      const int n = wave_n * WN + nt * 16 + r;
      bf[nt] = lds_b[cb][n * CPR + ((sub * 4 + q) ^ swz_b(n))];
    }
  };
  auto read_a = [&](int cb, int sub, int mt) {
    const int row = wave_m * WM + mt * 16 + r;
    return lds_a[cb][row * CPR + ((sub * 4 + q) ^ swz_a(row))];
  };
  // stage from buffer cb; the next stage's global data (already requested) is written to
  // buffer wb during the second 32-k half, one nibble of the dequant per A fragment
  auto step = [&](int cb, int wb) {
    u32x4 bf[NTL];
    u32x4 af[2];
    read_b(cb, 0, bf);
    af[0] = read_a(cb, 0, 0);
#pragma unroll
    for (int mt = 0; mt < MTL; ++mt) {
      if (mt + 1 < MTL) af[(mt + 1) & 1] = read_a(cb, 0, mt + 1);
      mfma_sub(cb, 0, mt, bf, af[mt & 1]);
    }
    __builtin_amdgcn_sched_barrier(0);
    read_b(cb, 1, bf);
    af[0] = read_a(cb, 1, 0);
    uint32_t lo[2], hi[2];
    lo[0] = pair_lo(braw[0], braw[1]);
    hi[0] = pair_hi(braw[0], braw[1]);
    lo[1] = pair_lo(braw[2], braw[3]);
    hi[1] = pair_hi(braw[2], braw[3]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int mt = 0; mt < MTL; ++mt) {
      if (mt + 1 < MTL) af[(mt + 1) & 1] = read_a(cb, 1, mt + 1);
      mfma_sub(cb, 1, mt, bf, af[mt & 1]);
      write_b_nib(wb, mt & 7, lo, hi);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // prologue: stage 0 into buffer 0, stage 1's weights in registers
  dma_a(0, 0);
  load_b(0);
#pragma unroll
  for (int j = 0; j < 4; ++j) braw[j] = bnext[j];
  bsz = bsznext;
  load_b(1);
  {
    uint32_t lo[2], hi[2];
    lo[0] = pair_lo(braw[0], braw[1]);
    hi[0] = pair_hi(braw[0], braw[1]);
    lo[1] = pair_lo(braw[2], braw[3]);
    hi[1] = pair_hi(braw[2], braw[3]);
#pragma unroll
    for (int I = 0; I < 8; ++I) write_b_nib(0, I, lo, hi);
  }
  AWQ_WAIT_VMCNT0();
#pragma unroll
  for (int j = 0; j < 4; ++j) braw[j] = bnext[j];
  bsz = bsznext;
  __syncthreads();
  // iteration s: request stage s + 1's activations (into the buffer stage s - 1 used) and
  // stage s + 2's weights, compute stage s from buffer s & 1 and, in its second half, write
  // stage s + 1's weights (held in registers since the last iteration) into the other buffer
  // (after the last stage into a buffer nobody reads); one barrier per 64-k stage, after this
  // wave's loads have landed
  for (int s = 0; s < nst; ++s) {
    if (s + 1 < nst) dma_a(s + 1, (s & 1) ^ 1);
    load_b(s + 2);
    step(s & 1, (s & 1) ^ 1);
    AWQ_WAIT_VMCNT0();
#pragma unroll
    for (int j = 0; j < 4; ++j) braw[j] = bnext[j];
    bsz = bsznext;
    __syncthreads();
  }

  // Epilogue through LDS (the k loop's last barrier has passed, so every stage buffer is free):
  // lane (q, r) holds acc[mt][nt][v] = C[wave_m WM + 16 mt + 4 q + v][wave_n WN + 16 nt + r] of
  // the tile; each value (+ bias, rounded once) goes to the row-major fp16 tile in LDS, whose
  // 16-byte chunks are XOR-swizzled by row, and the block then writes whole rows with 16-byte
  // stores (instead of 2-byte stores scattered over 4 rows each).
  constexpr int CCH = BN / 8;  // 16-byte chunks per output row
  auto c_chunk = [&](int row, int ch) { return ch ^ (row & 15 & (CCH - 1)); };
  __attribute__((address_space(3))) uint16_t* cl = (__attribute__((address_space(3))) uint16_t*)(uintptr_t)(uint32_t)(
      uintptr_t)(__attribute__((address_space(3))) u32x4*)&lds_all[0];
#pragma unroll
  for (int nt = 0; nt < NTL; ++nt) {
    const int cc = wave_n * WN + nt * 16 + r;  // tile column
    const int colg = n0 + cc;
    const float bv = (p.bias && colg < p.N) ? load_bias(p.bias, p.bias_dtype, colg) : 0.0f;
#pragma unroll
    for (int mt = 0; mt < MTL; ++mt) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = wave_m * WM + mt * 16 + 4 * q + v;
        cl[row * BN + c_chunk(row, cc >> 3) * 8 + (cc & 7)] = to_bits<T>(acc[mt][nt][v] + bv);
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
    const u32x4 val = lds_all[row * CCH + c_chunk(row, ch)];
    if (grow < p.M && gcol < p.N) *(u32x4*)(p.c + (int64_t)grow * p.ldc + gcol) = val;
  }
}

}  // namespace awq

namespace awq_host {
using namespace awq;

// 256-column tiles unless that leaves a CU without a block
template <bool SEQ, bool ZP, typename T, bool FAST>
static void launch_prefill_t(const GemmArgs& a, int sbf, hipStream_t st) {
  const int tm = (int)cdiv(a.M, kPBM);
  const int tn4 = (int)cdiv(a.N, 256);
  if ((int64_t)tm * tn4 >= num_cus()) {
    hipLaunchKernelGGL((prefill_kn_kernel<4, SEQ, ZP, T, FAST>), dim3(tm * tn4), dim3(512), 0, st, a, sbf, tm, tn4);
  } else {
    const int tn2 = (int)cdiv(a.N, 128);
    hipLaunchKernelGGL((prefill_kn_kernel<2, SEQ, ZP, T, FAST>), dim3(tm * tn2), dim3(256), 0, st, a, sbf, tm, tn2);
  }
}

template <bool SEQ, bool ZP>
static void dispatch(const GemmArgs& a, int act, int sdt, hipStream_t st) {
  const int sbf = (sdt == AWQ_DTYPE_BF16) ? 1 : 0;
  if (act == AWQ_DTYPE_F16) {
    if (sdt == AWQ_DTYPE_F16) launch_prefill_t<SEQ, ZP, f16, true>(a, sbf, st);
    else launch_prefill_t<SEQ, ZP, f16, false>(a, sbf, st);
  } else {
    launch_prefill_t<SEQ, ZP, bf16, false>(a, sbf, st);
  }
}

bool launch_prefill(const GemmArgs& a, bool seq, bool zp, int act, int sdt, hipStream_t st) {
  if (seq) {
    if (zp) dispatch<true, true>(a, act, sdt, st);
    else dispatch<true, false>(a, act, sdt, st);
  } else {
    if (zp) dispatch<false, true>(a, act, sdt, st);
    else dispatch<false, false>(a, act, sdt, st);
  }
  return true;
}

}  // namespace awq_host
