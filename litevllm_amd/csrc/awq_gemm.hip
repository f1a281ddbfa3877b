// Prefill GEMM (M > 32) for the KN layouts (qweight [K, N/8]) on gfx950: the role of
// _awq_native_tiled_gemm_autotuned (vllm/kernels/triton/awq_fused_gemm.py:2296-2392).
//
//  * Block tile 256 (M) x 64 NWN (N), k-stages of 32, 2 x NWN waves, wave tile 128 x 64:
//    8 x 4 accumulators of v_mfma_f32_16x16x32_{f16,bf16} per wave.  NWN = 4 (256 columns,
//    one 512-thread block per CU) halves the activation traffic per flop of NWN = 2.
//  * Each k-stage the block copies its activation tile into LDS and dequantizes its weight
//    tile once (every thread two packed words of two k-adjacent rows, exact (q - z) * s) into
//    LDS as [n][k] half values, so every wave reads both MFMA operands with 16-byte LDS loads
//    and no weight is dequantized twice in a block.
//  * LDS is double-buffered and the next stage's global loads ride in registers, so one
//    barrier per stage separates writing stage s + 1 from reading stage s.
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

// chunk swizzle of a 64-byte LDS row (four 16-byte chunks)
__device__ __forceinline__ int swz(int row) { return ((row >> 1) ^ (row >> 3)) & 3; }

constexpr int kPBM = 256, kPBK = 32;

template <int NWN, bool SEQ, bool ZP, typename T, bool FAST>
__global__ void __launch_bounds__(128 * NWN, 2) prefill_kn_kernel(const GemmArgs p, int scale_bf16, int tiles_m,
                                                               int tiles_n) {
  constexpr int NT = 128 * NWN;  // threads
  constexpr int BM = kPBM, BN = 64 * NWN, BK = kPBK;
  constexpr int WM = 128, WN = 64;
  constexpr int MTL = WM / 16, NTL = WN / 16;
  constexpr int ACH = BM * BK / 8 / NT;  // 16-byte activation chunks per thread per stage
  constexpr int BW = BN / 8;             // packed words per row of the tile
  __shared__ u32x4 lds_a[2][BM * BK / 8];
  __shared__ u32x4 lds_b[2][BN * BK / 8];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
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
  // dequant assignment: packed word bw of the tile, k-rows 2 rp and 2 rp + 1 of the stage
  const int bw = tid % BW, rp = tid / BW;
  const int bword = (n0 >> 3) + bw;
  const int bwld = bword < NW ? bword : NW - 1;  // columns past N are computed, never stored

  f32x4 acc[MTL][NTL];
#pragma unroll
  for (int mt = 0; mt < MTL; ++mt)
#pragma unroll
    for (int nt = 0; nt < NTL; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nst = p.K / BK;
  const MagicK mk = magic_consts();
  u32x4 areg[ACH];
  uint32_t b0, b1;
  WordSZ bsz;
  auto load = [&](int s) {
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int c = tid + NT * i;
      const int row = c >> 2, ch = c & 3;
      const int gr = min(m0 + row, p.M - 1);
      areg[i] = *(const u32x4*)(p.a + (int64_t)gr * p.lda + s * BK + ch * 8);
    }
    const int64_t k = (int64_t)s * BK + 2 * rp;
    b0 = __builtin_nontemporal_load(p.qw + k * NW + bwld);
    b1 = __builtin_nontemporal_load(p.qw + (k + 1) * NW + bwld);
    bsz = load_sz<ZP>(p, (s * BK) / p.G, bwld);
  };
  auto write = [&](int buf) {
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int c = tid + NT * i;
      const int row = c >> 2, ch = c & 3;
      lds_a[buf][row * 4 + (ch ^ swz(row))] = areg[i];
    }
    ColConst cc[8];
    prep_consts<SEQ, FAST>(bsz, scale_bf16 != 0, cc);
    const uint32_t lo = pair_lo(b0, b1), hi = pair_hi(b0, b1);
    uint32_t* const lb = (uint32_t*)lds_b[buf];
#define AWQ_PF_NIB(I)                                                                      \
    {                                                                                      \
      const uint32_t v = deq2<FAST, T>(magic_bits<(I) & 3>((I) < 4 ? lo : hi, mk), cc[I]); \
      const int n = 8 * bw + nib_col<SEQ>(I);                                              \
      lb[(n * 4 + ((rp >> 2) ^ swz(n))) * 4 + (rp & 3)] = v;                               \
    }
    AWQ_PF_NIB(0) AWQ_PF_NIB(1) AWQ_PF_NIB(2) AWQ_PF_NIB(3)
    AWQ_PF_NIB(4) AWQ_PF_NIB(5) AWQ_PF_NIB(6) AWQ_PF_NIB(7)
#undef AWQ_PF_NIB
  };
  auto compute = [&](int buf) {
    u32x4 bf[NTL];
#pragma unroll
    for (int nt = 0; nt < NTL; ++nt) {
      const int n = wave_n * WN + nt * 16 + r;
      bf[nt] = lds_b[buf][n * 4 + (q ^ swz(n))];
    }
#pragma unroll
    for (int mt = 0; mt < MTL; ++mt) {
      const int row = wave_m * WM + mt * 16 + r;
      const u32x4 af = lds_a[buf][row * 4 + (q ^ swz(row))];
#pragma unroll
      for (int nt = 0; nt < NTL; ++nt) acc[mt][nt] = MfmaOp<T>::run(af, bf[nt], acc[mt][nt]);
    }
  };

  load(0);
  write(0);
  if (nst > 1) load(1);
  __syncthreads();
  for (int s = 0; s < nst; ++s) {
    compute(s & 1);
    if (s + 1 < nst) write((s + 1) & 1);
    if (s + 2 < nst) load(s + 2);
    __syncthreads();
  }

  // lane (q, r) holds acc[mt][nt][v] = C[m0 + wave_m*WM + mt*16 + 4q + v][n0 + wave_n*WN + nt*16 + r]
#pragma unroll
  for (int nt = 0; nt < NTL; ++nt) {
    const int col = n0 + wave_n * WN + nt * 16 + r;
    if (col >= p.N) continue;
    const float bv = p.bias ? load_bias(p.bias, p.bias_dtype, col) : 0.0f;
#pragma unroll
    for (int mt = 0; mt < MTL; ++mt) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = m0 + wave_m * WM + mt * 16 + 4 * q + v;
        if (row < p.M) p.c[(int64_t)row * p.ldc + col] = to_bits<T>(acc[mt][nt][v] + bv);
      }
    }
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
