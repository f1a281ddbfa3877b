// Prefill GEMM (M > 32) for the KN layouts (qweight [K, N/8]) on gfx950: the role of
// _awq_native_tiled_gemm_autotuned (vllm/kernels/triton/awq_fused_gemm.py:2296-2392) with
// the weight dequantized once per wave into MFMA operand layout.
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


// Prefill GEMM kernel, KN layouts.  Block tile BM x 256, 4 waves in a 2 x 2 grid, wave tile
// (BM/2) x 128.  A (activations) goes through LDS in 64-wide k stages (double buffered,
// 16-byte chunks XOR-swizzled by row); each wave reads its own 16 weight words per row
// from global memory and dequantizes them into MFMA operands in registers.
template <int BM, bool SEQ, bool ZP, typename T, bool FAST>
__global__ void __launch_bounds__(256) gemm_kn_kernel(const GemmArgs p, int scale_bf16,
                                                      int tiles_m, int tiles_n) {
  constexpr int BK = 64;
  constexpr int WM = BM / 2;
  constexpr int MTL = WM / 16;               // m-tiles per wave
  constexpr int ACH = BM * BK / 8 / 256;     // 16-byte A chunks per thread per stage
  __shared__ u32x4 lds_a[2][BM * BK / 8];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int q = lane >> 4, r = lane & 15;
  const int wave_m = wave >> 1, wave_n = wave & 1;

  // XCD-aware tile order: blocks are dealt round-robin to the 8 XCDs; give each XCD a
  // contiguous range of tiles (row-tile major) so blocks sharing an A row-tile share an L2.
  const int ntiles = tiles_m * tiles_n;
  int bid = blockIdx.x;
  if ((ntiles & 7) == 0) bid = (bid & 7) * (ntiles >> 3) + (bid >> 3);
  const int tm = bid / tiles_n, tn = bid - tm * tiles_n;
  const int m0 = tm * BM, n0 = tn * 256;

  const int NW = p.N >> 3;
  const int word = (n0 >> 3) + wave_n * 16 + r;
  const bool wvalid = word < NW;
  const int wld = wvalid ? word : 0;

  f32x4 acc[MTL][8];
#pragma unroll
  for (int mt = 0; mt < MTL; ++mt)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[mt][i] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nst = p.K / BK;
  u32x4 areg[ACH];
  auto load_a = [&](int st) {
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int c = tid + 256 * i;
      const int row = c >> 3, ch = c & 7;
      const int gr = min(m0 + row, p.M - 1);
      areg[i] = *(const u32x4*)(p.a + (int64_t)gr * p.lda + st * BK + ch * 8);
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int c = tid + 256 * i;
      const int row = c >> 3, ch = c & 7;
      lds_a[buf][row * 8 + (ch ^ (row & 7))] = areg[i];
    }
  };
  uint32_t braw[2][8];
  WordSZ bsz[2];
  auto load_b = [&](int st, uint32_t (&dst)[2][8], WordSZ (&szd)[2]) {
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        dst[sub][j] = __builtin_nontemporal_load(p.qw + (int64_t)(st * BK + sub * 32 + 8 * q + j) * NW + wld);
      szd[sub] = load_sz<ZP>(p, (st * BK + sub * 32) / p.G, wld);
    }
  };

  ColConst cc[8];
  int cur_g = -1;
  const MagicK mk = magic_consts();

  load_a(0);
  store_a(0);
  load_b(0, braw, bsz);
  __syncthreads();

  for (int st = 0; st < nst; ++st) {
    const int buf = st & 1;
    uint32_t bnext[2][8];
    WordSZ sznext[2];
    if (st + 1 < nst) {
      load_a(st + 1);
      load_b(st + 1, bnext, sznext);
    }
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int g = (st * BK + sub * 32) / p.G;
      if (g != cur_g) {
        cur_g = g;
        prep_consts<SEQ, FAST>(bsz[sub], scale_bf16 != 0, cc);
      }
      u32x4 af[MTL];
#pragma unroll
      for (int mt = 0; mt < MTL; ++mt) {
        const int row = wave_m * WM + mt * 16 + r;
        const int ch = sub * 4 + q;
        af[mt] = lds_a[buf][row * 8 + (ch ^ (row & 7))];
      }
      uint32_t mlo[4], mhi[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        mlo[u] = pair_lo(braw[sub][2 * u], braw[sub][2 * u + 1]);
        mhi[u] = pair_hi(braw[sub][2 * u], braw[sub][2 * u + 1]);
      }
#define AWQ_GEMM_NIB(I)                                                          \
      {                                                                          \
        const u32x4 bop = rows_operand<I, FAST, T>(mlo, mhi, cc[I], mk);         \
        _Pragma("unroll") for (int mt = 0; mt < MTL; ++mt)                       \
            acc[mt][I] = MfmaOp<T>::run(af[mt], bop, acc[mt][I]);                \
      }
      AWQ_GEMM_NIB(0) AWQ_GEMM_NIB(1) AWQ_GEMM_NIB(2) AWQ_GEMM_NIB(3)
      AWQ_GEMM_NIB(4) AWQ_GEMM_NIB(5) AWQ_GEMM_NIB(6) AWQ_GEMM_NIB(7)
#undef AWQ_GEMM_NIB
    }
    if (st + 1 < nst) {
      store_a(buf ^ 1);
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
#pragma unroll
        for (int j = 0; j < 8; ++j) braw[sub][j] = bnext[sub][j];
        bsz[sub] = sznext[sub];
      }
    }
    __syncthreads();
  }

  // lane (q, r) holds acc[mt][i][v] = C[row m0 + wave_m*WM + mt*16 + 4q + v][8*word + nib_col(i)]
  if (!wvalid) return;
  float bv[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) bv[c] = p.bias ? load_bias(p.bias, p.bias_dtype, 8 * word + c) : 0.0f;
#pragma unroll
  for (int mt = 0; mt < MTL; ++mt) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = m0 + wave_m * WM + mt * 16 + 4 * q + v;
      if (row >= p.M) continue;
      float o[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) o[c] = acc[mt][col_nib<SEQ>(c)][v] + bv[c];
      u32x4 st;
      st[0] = pack2<T>(o[0], o[1]);
      st[1] = pack2<T>(o[2], o[3]);
      st[2] = pack2<T>(o[4], o[5]);
      st[3] = pack2<T>(o[6], o[7]);
      *(u32x4*)(p.c + (int64_t)row * p.ldc + 8 * word) = st;
    }
  }
}


}  // namespace awq

namespace awq_host {
using namespace awq;

template <int BM, bool SEQ, bool ZP, typename T, bool FAST>
static void launch_gemm_t(const GemmArgs& a, int sbf, hipStream_t st) {
  const int tm = (int)cdiv(a.M, BM), tn = (int)cdiv(a.N, 256);
  hipLaunchKernelGGL((gemm_kn_kernel<BM, SEQ, ZP, T, FAST>), dim3(tm * tn), dim3(256), 0, st, a,
                     sbf, tm, tn);
}

static int pick_bm(int64_t M, int64_t N) {
  const int64_t slots = num_cus();
  auto fill = [&](int64_t bm) {
    const int64_t blocks = cdiv(M, bm) * cdiv(N, 256);
    return (double)blocks / ((double)cdiv(blocks, slots) * (double)slots);
  };
  if (M >= 256 && fill(256) >= 0.99 * fill(128)) return 256;
  return 128;
}

template <bool SEQ, bool ZP, typename T, bool FAST>
static void launch_gemm_sel(const GemmArgs& a, int sbf, hipStream_t st) {
  if (pick_bm(a.M, a.N) == 256) launch_gemm_t<256, SEQ, ZP, T, FAST>(a, sbf, st);
  else launch_gemm_t<128, SEQ, ZP, T, FAST>(a, sbf, st);
}

template <bool SEQ, bool ZP>
static void dispatch(const GemmArgs& a, int act, int sdt, hipStream_t st) {
  const int sbf = (sdt == AWQ_DTYPE_BF16) ? 1 : 0;
  if (act == AWQ_DTYPE_F16) {
    if (sdt == AWQ_DTYPE_F16) launch_gemm_sel<SEQ, ZP, f16, true>(a, sbf, st);
    else launch_gemm_sel<SEQ, ZP, f16, false>(a, sbf, st);
  } else {
    launch_gemm_sel<SEQ, ZP, bf16, false>(a, sbf, st);
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
