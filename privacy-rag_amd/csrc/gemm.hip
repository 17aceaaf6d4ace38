// Party-local share GEMM over Z_2^64 on the i8 matrix cores of gfx950.
//
//   y[m][n] = ((sum_k x[m][k] * w[n][k]) << s_n)  mod 2^mask_bits
//
// (bfv_matrix.inc:101-105 / 156-160 / 177-182: the reference runs this as a
// scalar triple loop on the protocol thread.)
//
// Exactness.  Each u64 share is split into its 8 bytes b_d and re-centred as
// signed digits a_d = b_d - 128 (one XOR with 0x80 per byte), so that
//   x = sum_d (a_d + 128) 256^d
//   sum_k x w = sum_d 256^d (sum_k a_d w)  +  0x8080808080808080 * sum_k w   (mod 2^64).
// Every digit product a_d * w fits i8 x i8, and each column of partial sums
// fits the i32 accumulator (|a_d w| <= 2^14, K < 2^17).  int32 weights in
// [-0x808080, 0x7F7F7F] (the reference f12 domain is |w| <= 2^20) are split
// into three balanced signed bytes w = sum_e w_e 256^e and run as one pass per
// weight byte, each pass shifting its contribution by 8e and accumulating
// mod 2^64.
//
// Tiling.  One MFMA v_mfma_i32_32x32x32_i8 covers 32 "digit rows" = 4 share
// rows x 8 digits, ordered so that the 16 accumulator registers of a lane hold
// all 8 digits of 2 share rows for its column (32x32 accumulator layout: lane l,
// register r -> column l%32, row 8(r/4) + 4(l/32) + r%4).  The digit sum is
// therefore formed in registers with no cross-lane traffic.  A workgroup of 4
// waves computes 32 share rows x 128 columns; each wave 16 rows x 64 columns
// (8 MFMAs per 32-wide K step).  Shares are staged in LDS as 8 digit planes
// (byte transpose with v_perm), weights as int8 rows; both with an 80-byte row
// pitch so the 16-byte operand reads are bank-conflict free.
#include "kernels.hpp"

namespace praghip {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kBM = 32, kBN = 128, kBK = 64, kPitch = 80, kThreads = 256;

// o_d byte e = a_e byte d, for four dwords a0..a3.
__device__ __forceinline__ void transpose4(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3, uint32_t& o0,
                                           uint32_t& o1, uint32_t& o2, uint32_t& o3) {
  const uint32_t p0 = __builtin_amdgcn_perm(a1, a0, 0x05010400u);
  const uint32_t p1 = __builtin_amdgcn_perm(a1, a0, 0x07030602u);
  const uint32_t p2 = __builtin_amdgcn_perm(a3, a2, 0x05010400u);
  const uint32_t p3 = __builtin_amdgcn_perm(a3, a2, 0x07030602u);
  o0 = __builtin_amdgcn_perm(p2, p0, 0x05040100u);
  o1 = __builtin_amdgcn_perm(p2, p0, 0x07060302u);
  o2 = __builtin_amdgcn_perm(p3, p1, 0x05040100u);
  o3 = __builtin_amdgcn_perm(p3, p1, 0x07060302u);
}

// Balanced signed byte e (e < 3) of a weight in [-0x808080, 0x7F7F7F].
__device__ __forceinline__ int weight_digit(int w, int e) {
  for (int i = 0; i < e; ++i) {
    const int lo = (int)(int8_t)(w & 0xff);
    w = (w - lo) >> 8;
  }
  return (int)(int8_t)(w & 0xff);
}

// Global tile of one K step held in registers: the share loader's 8 u64 and
// the weight loader's 32 weight bytes (as 8 words).
struct TileRegs {
  uint64_t xs[8];
  uint32_t wb[8];
};

template <int WB>
__device__ __forceinline__ void load_tile(TileRegs& tr, const uint64_t* __restrict__ xrow, bool x_row_ok,
                                          const void* __restrict__ wv, size_t wrow_off, bool w_row_ok, int k0, int K,
                                          int ak, int wk, int wdigit, int w_vec) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int kk = k0 + ak + e;
    tr.xs[e] = (x_row_ok && kk < K) ? xrow[kk] : 0;
  }
  const int kk = k0 + wk;
  if (WB == 8) {
    const int8_t* wrow = static_cast<const int8_t*>(wv) + wrow_off;
    if (w_row_ok && kk + 32 <= K && w_vec) {
      const uint4 a = *reinterpret_cast<const uint4*>(wrow + kk);
      const uint4 b = *reinterpret_cast<const uint4*>(wrow + kk + 16);
      tr.wb[0] = a.x; tr.wb[1] = a.y; tr.wb[2] = a.z; tr.wb[3] = a.w;
      tr.wb[4] = b.x; tr.wb[5] = b.y; tr.wb[6] = b.z; tr.wb[7] = b.w;
    } else {
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        uint32_t word = 0;
#pragma unroll
        for (int bb = 0; bb < 4; ++bb) {
          const int kq = kk + 4 * q + bb;
          const uint32_t byte = (w_row_ok && kq < K) ? uint8_t(wrow[kq]) : 0u;
          word |= byte << (8 * bb);
        }
        tr.wb[q] = word;
      }
    }
  } else {
    const int32_t* wrow = static_cast<const int32_t*>(wv) + wrow_off;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      uint32_t word = 0;
#pragma unroll
      for (int bb = 0; bb < 4; ++bb) {
        const int kq = kk + 4 * q + bb;
        const int wvv = (w_row_ok && kq < K) ? wrow[kq] : 0;
        word |= uint32_t(uint8_t(weight_digit(wvv, wdigit))) << (8 * bb);
      }
      tr.wb[q] = word;
    }
  }
}

// Two workgroups per CU (two waves per SIMD, accumulators in VGPRs): while
// one waits on memory the other runs MFMAs.  Within a workgroup the next K
// step's global loads are issued before the current step's MFMAs.
template <int WB>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
    share_gemm_kernel(const uint64_t* __restrict__ x, const void* __restrict__ wv, const int8_t* __restrict__ shifts,
                      uint64_t* __restrict__ y, int M, int K, int N, uint64_t mask, int wdigit, int accumulate,
                      int w_vec) {
  __shared__ __attribute__((aligned(16))) uint8_t a_lds[8][kBM][kPitch];
  __shared__ __attribute__((aligned(16))) uint8_t w_lds[kBN][kPitch];
  __shared__ int csum[kThreads];

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;

  // share-tile loader: row ar, 8 consecutive k from ak
  const int ar = t >> 3, ak = (t & 7) * 8;
  // weight-tile loader: row wr, 32 consecutive k from wk
  const int wr = t >> 1, wk = (t & 1) * 32;
  int colsum = 0;

  // MFMA operand coordinates of this lane
  const int i = lane & 31, khalf = lane >> 5;
  const int a_row_in_block = 2 * ((i >> 2) & 1) + (i >> 4);
  const int a_digit = 4 * ((i >> 3) & 1) + (i & 3);

  v16i acc[4][2];
#pragma unroll
  for (int rb = 0; rb < 4; ++rb)
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) acc[rb][cb] = v16i{0};

  const bool x_row_ok = (m0 + ar) < M;
  const bool w_row_ok = (n0 + wr) < N;
  const uint64_t* xrow = x + size_t(m0 + ar) * K;
  const size_t wrow_off = size_t(n0 + wr) * K;

  TileRegs tr;
  load_tile<WB>(tr, xrow, x_row_ok, wv, wrow_off, w_row_ok, 0, K, ak, wk, wdigit, w_vec);
  for (int k0 = 0; k0 < K; k0 += kBK) {
    // ---- shares -> 8 offset-binary digit planes
    uint32_t d[16];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      d[2 * e] = uint32_t(tr.xs[e]) ^ 0x80808080u;
      d[2 * e + 1] = uint32_t(tr.xs[e] >> 32) ^ 0x80808080u;
    }
    uint32_t o[4][4];
    transpose4(d[0], d[2], d[4], d[6], o[0][0], o[0][1], o[0][2], o[0][3]);      // digits 0-3, k 0-3
    transpose4(d[8], d[10], d[12], d[14], o[1][0], o[1][1], o[1][2], o[1][3]);   // digits 0-3, k 4-7
    transpose4(d[1], d[3], d[5], d[7], o[2][0], o[2][1], o[2][2], o[2][3]);      // digits 4-7, k 0-3
    transpose4(d[9], d[11], d[13], d[15], o[3][0], o[3][1], o[3][2], o[3][3]);   // digits 4-7, k 4-7
#pragma unroll
    for (int dg = 0; dg < 4; ++dg) {
      *reinterpret_cast<uint2*>(&a_lds[dg][ar][ak]) = make_uint2(o[0][dg], o[1][dg]);
      *reinterpret_cast<uint2*>(&a_lds[dg + 4][ar][ak]) = make_uint2(o[2][dg], o[3][dg]);
    }
    // ---- weights (digit `wdigit` of each) -> int8 rows
#pragma unroll
    for (int q = 0; q < 8; ++q) colsum = __builtin_amdgcn_sdot4(int(tr.wb[q]), 0x01010101, colsum, false);
    *reinterpret_cast<uint4*>(&w_lds[wr][wk]) = make_uint4(tr.wb[0], tr.wb[1], tr.wb[2], tr.wb[3]);
    *reinterpret_cast<uint4*>(&w_lds[wr][wk + 16]) = make_uint4(tr.wb[4], tr.wb[5], tr.wb[6], tr.wb[7]);
    __syncthreads();
    // ---- next step's loads, in flight during the MFMAs
    if (k0 + kBK < K) load_tile<WB>(tr, xrow, x_row_ok, wv, wrow_off, w_row_ok, k0 + kBK, K, ak, wk, wdigit, w_vec);

    // ---- MFMA over the two 32-wide K steps
#pragma unroll
    for (int ks = 0; ks < kBK / 32; ++ks) {
      const int kb = ks * 32 + khalf * 16;
      v4i bop[2];
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) bop[cb] = *reinterpret_cast<const v4i*>(&w_lds[wn * 64 + cb * 32 + i][kb]);
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
        const v4i aop = *reinterpret_cast<const v4i*>(&a_lds[a_digit][wm * 16 + rb * 4 + a_row_in_block][kb]);
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
          acc[rb][cb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop, bop[cb], acc[rb][cb], 0, 0, 0);
      }
    }
    __syncthreads();
  }

  // ---- epilogue: column sums, digit recombination, shift, mask
  csum[t] = colsum;
  __syncthreads();
  const int shift_e = 8 * wdigit;
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
    const int cl = wn * 64 + cb * 32 + i;
    const int col = n0 + cl;
    if (col >= N) continue;
    const int64_t s_n = int64_t(csum[2 * cl]) + int64_t(csum[2 * cl + 1]);
    const uint64_t corr = 0x8080808080808080ull * uint64_t(s_n);
    const int sh = shift_e + (shifts ? int(shifts[col]) : 0);
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const int row = m0 + wm * 16 + rb * 4 + 2 * khalf + a;
        if (row >= M) continue;
        uint64_t v = corr;
#pragma unroll
        for (int dg = 0; dg < 8; ++dg) v += uint64_t(int64_t(acc[rb][cb][8 * a + dg])) << (8 * dg);
        v = sh < 64 ? (v << sh) : 0;
        uint64_t* dst = y + size_t(row) * N + col;
        if (accumulate) v += *dst;
        *dst = v & mask;
      }
    }
  }
}

// ------------------------------------------------------------- VALU form
// The same product with VALU dot products instead of the matrix cores: the
// tiles are staged exactly as in share_gemm_kernel (digit planes of the
// offset-binary share bytes, int8 weight rows), and each thread forms a 4 x 4
// block of outputs with v_dot4_i32_i8, one per (row, column, digit) and four
// k.  It exists as the measured alternative to the MFMA kernels (int8
// weights).
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
    share_gemm_valu_kernel(const uint64_t* __restrict__ x, const int8_t* __restrict__ w,
                           const int8_t* __restrict__ shifts, uint64_t* __restrict__ y, int M, int K, int N,
                           uint64_t mask, int w_vec) {
  __shared__ __attribute__((aligned(16))) uint8_t a_lds[8][kBM][kPitch];
  __shared__ __attribute__((aligned(16))) uint8_t w_lds[kBN][kPitch];
  __shared__ int csum[kThreads];
  const int t = threadIdx.x;
  const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;
  const int ar = t >> 3, ak = (t & 7) * 8, wr = t >> 1, wk = (t & 1) * 32;
  const int rg = t >> 5, cg = t & 31;  // rows rg + 8i, columns cg + 32j
  int colsum = 0;
  int acc[4][4][8];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int d = 0; d < 8; ++d) acc[i][j][d] = 0;
  const bool x_row_ok = (m0 + ar) < M, w_row_ok = (n0 + wr) < N;
  const uint64_t* xrow = x + size_t(m0 + ar) * K;
  const size_t wrow_off = size_t(n0 + wr) * K;
  TileRegs tr;
  load_tile<8>(tr, xrow, x_row_ok, w, wrow_off, w_row_ok, 0, K, ak, wk, 0, w_vec);
  for (int k0 = 0; k0 < K; k0 += kBK) {
    uint32_t d[16];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      d[2 * e] = uint32_t(tr.xs[e]) ^ 0x80808080u;
      d[2 * e + 1] = uint32_t(tr.xs[e] >> 32) ^ 0x80808080u;
    }
    uint32_t o[4][4];
    transpose4(d[0], d[2], d[4], d[6], o[0][0], o[0][1], o[0][2], o[0][3]);
    transpose4(d[8], d[10], d[12], d[14], o[1][0], o[1][1], o[1][2], o[1][3]);
    transpose4(d[1], d[3], d[5], d[7], o[2][0], o[2][1], o[2][2], o[2][3]);
    transpose4(d[9], d[11], d[13], d[15], o[3][0], o[3][1], o[3][2], o[3][3]);
#pragma unroll
    for (int dg = 0; dg < 4; ++dg) {
      *reinterpret_cast<uint2*>(&a_lds[dg][ar][ak]) = make_uint2(o[0][dg], o[1][dg]);
      *reinterpret_cast<uint2*>(&a_lds[dg + 4][ar][ak]) = make_uint2(o[2][dg], o[3][dg]);
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) colsum = __builtin_amdgcn_sdot4(int(tr.wb[q]), 0x01010101, colsum, false);
    *reinterpret_cast<uint4*>(&w_lds[wr][wk]) = make_uint4(tr.wb[0], tr.wb[1], tr.wb[2], tr.wb[3]);
    *reinterpret_cast<uint4*>(&w_lds[wr][wk + 16]) = make_uint4(tr.wb[4], tr.wb[5], tr.wb[6], tr.wb[7]);
    __syncthreads();
#pragma unroll 1
    for (int kk = 0; kk < kBK; kk += 4) {
      int wv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) wv[j] = *reinterpret_cast<const int*>(&w_lds[cg + 32 * j][kk]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int dg = 0; dg < 8; ++dg) {
          const int xv = *reinterpret_cast<const int*>(&a_lds[dg][rg + 8 * i][kk]);
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j][dg] = __builtin_amdgcn_sdot4(xv, wv[j], acc[i][j][dg], false);
        }
      }
    }
    __syncthreads();
    // the next step's tile is loaded after the dot products (the 128
    // accumulators leave no registers to hold it during them)
    if (k0 + kBK < K) load_tile<8>(tr, xrow, x_row_ok, w, wrow_off, w_row_ok, k0 + kBK, K, ak, wk, 0, w_vec);
  }
  csum[t] = colsum;
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int cl = cg + 32 * j, col = n0 + cl;
    if (col >= N) continue;
    const int64_t s_n = int64_t(csum[2 * cl]) + int64_t(csum[2 * cl + 1]);
    const uint64_t corr = 0x8080808080808080ull * uint64_t(s_n);
    const int sh = shifts ? int(shifts[col]) : 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = m0 + rg + 8 * i;
      if (row >= M) continue;
      uint64_t v = corr;
#pragma unroll
      for (int dg = 0; dg < 8; ++dg) v += uint64_t(int64_t(acc[i][j][dg])) << (8 * dg);
      v = sh < 64 ? (v << sh) : 0;
      y[size_t(row) * N + col] = v & mask;
    }
  }
}

hipError_t launch_share_gemm_valu(const uint64_t* x, const int8_t* w, const int8_t* shifts, uint64_t* y, int M,
                                  int K, int N, int mask_bits, hipStream_t s) {
  const uint64_t mask = mask_bits >= 64 ? ~0ull : ((1ull << mask_bits) - 1);
  const int w_vec = (K % 16 == 0) && (reinterpret_cast<uintptr_t>(w) % 16 == 0);
  const dim3 grid((N + kBN - 1) / kBN, (M + kBM - 1) / kBM);
  hipLaunchKernelGGL(share_gemm_valu_kernel, grid, dim3(kThreads), 0, s, x, w, shifts, y, M, K, N, mask, w_vec);
  return hipGetLastError();
}

// ---------------------------------------------------------------- DMA path
// For K % 64 == 0 and int8 weights (16-byte aligned x, w): the raw tiles go
// from global memory straight into a two-stage LDS ring with
// global_load_lds_dwordx4 (no registers, no wait until the stage is used), so
// the next K step's loads are in flight during the current step's MFMAs; two
// workgroups per CU overlap each other's waits as well.  Per step each thread
// turns 8 shares of the raw tile into the 8 digit planes (as above), and the
// weight tile is read by the MFMAs in place.
//
// LDS: raw shares [2][32 rows][512 B], weights [2][128 rows][64 B] with the
// 16-byte chunk index of row r stored at chunk ^ (r & 3) (conflict-free
// operand reads without padding, which DMA cannot insert), digit planes
// [8][34][80 B]: two spare rows per plane make the plane stride 2720 bytes
// instead of 2560 (a multiple of the bank span), so the MFMA operand reads of
// one row across the 8 digits spread over the banks (measured 3-5% faster).
constexpr int kRawRow = kBK * 8;  // bytes of one raw share row per step

// 16 bytes per lane from global memory straight into LDS at M0 + lane * 16
// (global_load_lds_dwordx4).  Issued from inline asm, so the compiler adds no
// wait of its own for it: the caller waits with s_waitcnt vmcnt(0) before any
// wave reads what was loaded.
__device__ __forceinline__ void dma16(const void* src, void* lds_wave_base) {
  const unsigned lds = unsigned(reinterpret_cast<uintptr_t>((void __attribute__((address_space(3)))*)(lds_wave_base)));
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(__builtin_amdgcn_readfirstlane(lds)) : "memory");
}

// One K step of the DMA path on stage buffers (raw, wt); the next step's DMAs
// go to (raw_n, wt_n).  Distinct __shared__ objects per stage let the
// compiler see that this step's LDS reads do not depend on the DMAs just
// issued into the other stage (it would otherwise wait for them).
struct DmaCtx {
  const uint8_t* xsrc[4];
  const int8_t* wsrc[2];
  int wave, ar, ak, cl, ch, i, khalf, a_row_in_block, a_digit, wm, wn;
};

template <class RAW, class WT>
__device__ __forceinline__ void dma_issue(const DmaCtx& c, int k0, RAW& raw, WT& wt) {
#pragma unroll
  for (int j = 0; j < 4; ++j) dma16(c.xsrc[j] + size_t(k0) * 8, &raw[(2 * (4 * c.wave + j)) * kRawRow]);
#pragma unroll
  for (int j = 0; j < 2; ++j) dma16(c.wsrc[j] + k0, &wt[(16 * (2 * c.wave + j)) * kBK]);
}

template <class RAW, class WT, class RAWN, class WTN>
__device__ __forceinline__ void dma_step(const DmaCtx& c, bool next, int k_next, const RAW& raw, const WT& wt,
                                         RAWN& raw_n, WTN& wt_n, uint8_t (&a_lds)[8][kBM + 2][kPitch], int& colsum,
                                         v16i (&acc)[4][2]) {
  // this wave's DMAs for this step are done (none other is in flight yet);
  // after the barrier every wave's are, and the previous step's reads are over
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  if (next) dma_issue(c, k_next, raw_n, wt_n);
  // ---- raw shares -> 8 offset-binary digit planes
  {
    const uint4* rp = reinterpret_cast<const uint4*>(&raw[c.ar * kRawRow + c.ak * 8]);
    const uint4 q0 = rp[0], q1 = rp[1], q2 = rp[2], q3 = rp[3];
    uint32_t d[16] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w, q2.x, q2.y, q2.z, q2.w, q3.x, q3.y, q3.z, q3.w};
#pragma unroll
    for (int e = 0; e < 16; ++e) d[e] ^= 0x80808080u;
    uint32_t o[4][4];
    transpose4(d[0], d[2], d[4], d[6], o[0][0], o[0][1], o[0][2], o[0][3]);
    transpose4(d[8], d[10], d[12], d[14], o[1][0], o[1][1], o[1][2], o[1][3]);
    transpose4(d[1], d[3], d[5], d[7], o[2][0], o[2][1], o[2][2], o[2][3]);
    transpose4(d[9], d[11], d[13], d[15], o[3][0], o[3][1], o[3][2], o[3][3]);
#pragma unroll
    for (int dg = 0; dg < 4; ++dg) {
      *reinterpret_cast<uint2*>(&a_lds[dg][c.ar][c.ak]) = make_uint2(o[0][dg], o[1][dg]);
      *reinterpret_cast<uint2*>(&a_lds[dg + 4][c.ar][c.ak]) = make_uint2(o[2][dg], o[3][dg]);
    }
  }
  // ---- column sums of the weight tile
  {
    const uint8_t* wrow = &wt[c.cl * kBK];
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
      const uint4 v = *reinterpret_cast<const uint4*>(wrow + (((2 * c.ch + cc) ^ (c.cl & 3)) * 16));
      colsum = __builtin_amdgcn_sdot4(int(v.x), 0x01010101, colsum, false);
      colsum = __builtin_amdgcn_sdot4(int(v.y), 0x01010101, colsum, false);
      colsum = __builtin_amdgcn_sdot4(int(v.z), 0x01010101, colsum, false);
      colsum = __builtin_amdgcn_sdot4(int(v.w), 0x01010101, colsum, false);
    }
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  // ---- MFMA over the two 32-wide K steps
#pragma unroll
  for (int ks = 0; ks < kBK / 32; ++ks) {
    const int chunk = ks * 2 + c.khalf;  // logical 16-byte chunk of the weight rows
    v4i bop[2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int row = c.wn * 64 + cb * 32 + c.i;
      bop[cb] = *reinterpret_cast<const v4i*>(&wt[row * kBK + ((chunk ^ (row & 3)) * 16)]);
    }
    const int kb = ks * 32 + c.khalf * 16;
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const v4i aop = *reinterpret_cast<const v4i*>(&a_lds[c.a_digit][c.wm * 16 + rb * 4 + c.a_row_in_block][kb]);
#pragma unroll
      for (int cb = 0; cb < 2; ++cb)
        acc[rb][cb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop, bop[cb], acc[rb][cb], 0, 0, 0);
    }
  }
}

// Weight planes: w holds `planes` int8 matrices [planes][N][K], plane e the
// signed byte of weight digit e (planes = 1: int8 weights; 3: the pre-split
// f12 weights).  Workgroup z takes plane z / splits and K split z % splits;
// plane e's products enter y shifted by 8e.
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
    share_gemm_dma_kernel(const uint64_t* __restrict__ x, const int8_t* __restrict__ w,
                          const int8_t* __restrict__ shifts, uint64_t* __restrict__ y, int M, int K, int N,
                          uint64_t mask, int k_split, int splits) {
  const int plane = int(blockIdx.z) / splits, split_z = int(blockIdx.z) % splits;
  w += size_t(plane) * size_t(N) * size_t(K);
  __shared__ __attribute__((aligned(16))) uint8_t raw0[kBM * kRawRow];
  __shared__ __attribute__((aligned(16))) uint8_t raw1[kBM * kRawRow];
  __shared__ __attribute__((aligned(16))) uint8_t wt0[kBN * kBK];
  __shared__ __attribute__((aligned(16))) uint8_t wt1[kBN * kBK];
  __shared__ __attribute__((aligned(16))) uint8_t a_lds[8][kBM + 2][kPitch];
  __shared__ int csum[kThreads];

  const int t = threadIdx.x, lane = t & 63;
  DmaCtx c;
  c.wave = t >> 6;
  c.wm = c.wave >> 1;
  c.wn = c.wave & 1;
  c.ar = t >> 3;  // transposer: raw row ar, shares ak..ak+7
  c.ak = (t & 7) * 8;
  c.cl = t >> 1;  // column sum: weight row cl, half ch
  c.ch = t & 1;
  c.i = lane & 31;
  c.khalf = lane >> 5;
  c.a_row_in_block = 2 * ((c.i >> 2) & 1) + (c.i >> 4);
  c.a_digit = 4 * ((c.i >> 3) & 1) + (c.i & 3);
  const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;
  // DMA sources of this lane: 4 raw-share instructions (2 rows of 512 B each)
  // and 2 weight instructions (16 rows of 64 B each) per wave and step.
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = 2 * (4 * c.wave + j) + (lane >> 5);
    const int grow = min(m0 + row, M - 1);  // rows past M: any valid row, results dropped
    c.xsrc[j] = reinterpret_cast<const uint8_t*>(x + size_t(grow) * K) + (lane & 31) * 16;
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int row = 16 * (2 * c.wave + j) + (lane >> 2);
    const int grow = min(n0 + row, N - 1);
    const int ck = (lane & 3) ^ (row & 3);  // logical chunk stored at physical chunk lane & 3
    c.wsrc[j] = w + size_t(grow) * K + ck * 16;
  }
  int colsum = 0;
  v16i acc[4][2];
#pragma unroll
  for (int rb = 0; rb < 4; ++rb)
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) acc[rb][cb] = v16i{0};

  // split-K: workgroup z takes K steps [z k_split, (z+1) k_split); with more
  // than one split the partial products are added into y (zeroed first) by
  // 64-bit atomics, exact mod 2^64 in any order
  const int k_begin = split_z * k_split;
  const int steps = min(k_split, K - k_begin) / kBK;
  dma_issue(c, k_begin, raw0, wt0);
  for (int s = 0; s < steps; s += 2) {
    dma_step(c, s + 1 < steps, k_begin + (s + 1) * kBK, raw0, wt0, raw1, wt1, a_lds, colsum, acc);
    if (s + 1 < steps)
      dma_step(c, s + 2 < steps, k_begin + (s + 2) * kBK, raw1, wt1, raw0, wt0, a_lds, colsum, acc);
  }
  const bool split = gridDim.z > 1;

  // ---- epilogue: column sums, digit recombination, shift, mask
  csum[t] = colsum;
  __syncthreads();
  const int i = c.i, khalf = c.khalf, wm = c.wm, wn = c.wn;
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
    const int c2 = wn * 64 + cb * 32 + i;
    const int col = n0 + c2;
    if (col >= N) continue;
    const int64_t s_n = int64_t(csum[2 * c2]) + int64_t(csum[2 * c2 + 1]);
    const uint64_t corr = 0x8080808080808080ull * uint64_t(s_n);
    const int sh = 8 * plane + (shifts ? int(shifts[col]) : 0);
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const int row = m0 + wm * 16 + rb * 4 + 2 * khalf + a;
        if (row >= M) continue;
        uint64_t v = corr;
#pragma unroll
        for (int dg = 0; dg < 8; ++dg) v += uint64_t(int64_t(acc[rb][cb][8 * a + dg])) << (8 * dg);
        v = sh < 64 ? (v << sh) : 0;
        if (split)
          atomicAdd(reinterpret_cast<unsigned long long*>(y + size_t(row) * N + col), (unsigned long long)v);
        else
          y[size_t(row) * N + col] = v & mask;
      }
    }
  }
}

// y = 0 before a split-K product (keep = 0); y &= mask after one (mask_bits < 64).
__global__ void __launch_bounds__(256) gemm_clear_kernel(uint64_t* __restrict__ y, size_t n, uint64_t keep) {
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x)
    y[i] = keep ? (y[i] & keep) : 0;
}

// Pre-split weights: planes[e][i] = balanced signed byte e of w[i] (w in
// [-0x808080, 0x7F7F7F]), so that w = sum_e planes[e] 256^e.
__global__ void __launch_bounds__(256) weight_split_kernel(const int32_t* __restrict__ w, int8_t* __restrict__ planes,
                                                           size_t count) {
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += size_t(gridDim.x) * blockDim.x) {
    const int v = w[i];
#pragma unroll
    for (int e = 0; e < 3; ++e) planes[size_t(e) * count + i] = int8_t(weight_digit(v, e));
  }
}

hipError_t launch_weight_split(const int32_t* w, int8_t* planes, size_t count, hipStream_t s) {
  if (!count) return hipSuccess;
  const unsigned grid = unsigned(std::min<size_t>((count + 255) / 256, 8192));
  hipLaunchKernelGGL(weight_split_kernel, dim3(grid), dim3(256), 0, s, w, planes, count);
  return hipGetLastError();
}

hipError_t launch_share_gemm(const uint64_t* x, const void* w, int w_bits, const int8_t* shifts, uint64_t* y,
                             int M, int K, int N, int mask_bits, hipStream_t s) {
  const uint64_t mask = mask_bits >= 64 ? ~0ull : ((1ull << mask_bits) - 1);
  const dim3 grid((N + kBN - 1) / kBN, (M + kBM - 1) / kBM), block(kThreads);
  // 16-byte weight loads need 16-byte aligned rows
  const int w_vec = (K % 16 == 0) && (reinterpret_cast<uintptr_t>(w) % 16 == 0);
  if (w_bits == 8 || w_bits == 24) {
    const int planes = w_bits == 8 ? 1 : 3;
    if (K % kBK == 0 && w_vec && reinterpret_cast<uintptr_t>(x) % 16 == 0) {
      // Split K while the tiles fill fewer than 256 workgroups (one per CU;
      // N = 1024 at M = 512 gives 128 tiles) and each split keeps >= 8 steps:
      // measured 37 -> 26 us at 512x2048x1024 and 54 -> 33 us at 512x3072x1024,
      // while going on to two workgroups per CU was slower.
      const int tiles = int(grid.x * grid.y), ksteps = K / kBK;
      int splits = 1;
      while (splits < 4 && tiles * splits < 256 && ksteps / (splits * 2) >= 8) splits *= 2;
      const int k_split = (ksteps + splits - 1) / splits * kBK;
      splits = (K + k_split - 1) / k_split;
      const size_t words = size_t(M) * N;
      const unsigned fgrid = unsigned(std::min<size_t>((words + 255) / 256, 4096));
      // several planes or K splits add their partial products into y
      const bool atomic = splits * planes > 1;
      if (atomic) {
        hipLaunchKernelGGL(gemm_clear_kernel, dim3(fgrid), dim3(256), 0, s, y, words, 0ull);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
      }
      hipLaunchKernelGGL(share_gemm_dma_kernel, dim3(grid.x, grid.y, unsigned(splits * planes)), block, 0, s, x,
                         static_cast<const int8_t*>(w), shifts, y, M, K, N, mask, k_split, splits);
      hipError_t e = hipGetLastError();
      if (e == hipSuccess && atomic && mask != ~0ull) {
        hipLaunchKernelGGL(gemm_clear_kernel, dim3(fgrid), dim3(256), 0, s, y, words, mask);
        e = hipGetLastError();
      }
      return e;
    }
    // register-staged kernel, one launch per plane (plane e shifted by 8e,
    // accumulated into y after the first)
    for (int e = 0; e < planes; ++e) {
      const int8_t* we = static_cast<const int8_t*>(w) + size_t(e) * size_t(N) * size_t(K);
      hipLaunchKernelGGL((share_gemm_kernel<8>), grid, block, 0, s, x, we, shifts, y, M, K, N, mask, e, e > 0,
                         w_vec);
      const hipError_t err = hipGetLastError();
      if (err != hipSuccess) return err;
    }
    return hipSuccess;
  }
  for (int e = 0; e < 3; ++e) {
    hipLaunchKernelGGL((share_gemm_kernel<32>), grid, block, 0, s, x, w, shifts, y, M, K, N, mask, e, e > 0, 0);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  return hipSuccess;
}

}  // namespace praghip
