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
// from global memory straight into a three-stage LDS ring with
// global_load_lds_dwordx4 (no registers, no wait until the stage is used), so
// the next two K steps' loads are in flight during the current step's MFMAs;
// two workgroups per CU overlap each other's waits as well.  The MFMA share
// operands are read from the raw u64 tile with ds_read_b64_tr_b8, which hands
// every lane one byte position of eight words: with the eight words of a row
// k..k+7 as the source, lane i of each 8-lane half of a 16-lane group receives
// digit i of those eight shares (the byte transpose is done by the LDS read,
// with no VALU shuffle, no digit-plane copy and no second barrier per step).
//
// MFMA rows of one 32x32x32 product: lane l of the A operand is digit l % 8 of
// share row (l % 32) / 8, so a lane's 16 accumulator registers hold, for its
// column, digits 4(l/32)..4(l/32)+3 of four share rows; the two halves of the
// wave add their digit sums with one cross-half exchange.
//
// LDS: raw shares [3][32 rows][512 B] with the 16-byte chunk c of row r at
// chunk c ^ 4(r & 7) (each 8-word read of a row stays one 64-byte block, and
// the four rows of one read land on distinct banks), weights [3][128 rows][64 B]
// with chunk c of row r at c ^ wt_swizzle(r).  DMA writes 64 lanes x 16 bytes in
// order, so each lane loads the global chunk that belongs at its LDS slot.
constexpr int kRawRow = kBK * 8;  // bytes of one raw share row per step

// 16 bytes per lane from global memory straight into LDS at M0 + lane * 16
// (global_load_lds_dwordx4).  Issued from inline asm, so the compiler adds no
// wait of its own for it: the caller waits with s_waitcnt vmcnt(0) before any
// wave reads what was loaded.  The LDS DMA reads M0 one wait state after the
// scalar write that sets it (the compiler's own global_load_lds always leaves
// one instruction there); the compiler cannot see that dependency into the
// asm, so the asm starts with s_nop 0.
__device__ __forceinline__ void dma16(const void* src, void* lds_wave_base) {
  const unsigned lds = unsigned(reinterpret_cast<uintptr_t>((void __attribute__((address_space(3)))*)(lds_wave_base)));
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}

// Byte offset of share word k of raw row r in a stage buffer.
__device__ __forceinline__ int raw_offset(int r, int k) {
  return r * kRawRow + ((((k >> 1) ^ (4 * (r & 7)))) << 4) + ((k & 1) << 3);
}

// Chunk swizzle of weight row r (64-byte rows, four 16-byte chunks): 16-byte
// reads of 8 consecutive rows land on 8 distinct 16-byte bank slots of a
// 128-byte bank line, and those of rows r, r + 4, r + 8, r + 12 on 4 distinct
// slots of a 256-byte one (bits: 2 (r/4 % 2) + (r/2 % 2 ^ r/8 % 2)).
__device__ __forceinline__ int wt_swizzle(int r) { return 2 * ((r >> 2) & 1) + (((r >> 1) ^ (r >> 3)) & 1); }

typedef int v2i __attribute__((ext_vector_type(2)));

// Eight bytes of the LDS transpose read at byte offset `off` of `base`.
__device__ __forceinline__ v2i tr8(const uint8_t* base, int off) {
  return __builtin_amdgcn_ds_read_tr8_b64_v2i32((v2i __attribute__((address_space(3)))*)(base + off));
}

// One K step of the DMA path on stage buffers (raw, wt); the next step's DMAs
// go to (raw_n, wt_n).  Distinct __shared__ objects per stage let the
// compiler see that this step's LDS reads do not depend on the DMAs just
// issued into the other stage (it would otherwise wait for them).
struct DmaCtx {
  const uint8_t* xsrc[4];
  const int8_t* wsrc[3];
  int wave, i, khalf, wm, wn, tr_row, tr_k;
  // operand read offsets within a stage: share word run h (k + 8h) of row
  // block 0 at K step 0 is a_off[h]; row block rb, K step ks adds
  // 2048 rb + 256 (ks ^ (rb & 1)).  Weight chunk of K step ks for block 0 is
  // w_off[ks]; block cb adds 2048 cb.  (raw_offset and wt_swizzle, with the
  // lane-independent parts moved into immediates.)
  int a_off[2], w_off[2];
};

// CB 32-column blocks per wave: a workgroup tile is 32 share rows x 64 CB
// columns (waves 2 x 2, each 16 rows x 32 CB columns).
template <int CB, class RAW, class WT>
__device__ __forceinline__ void dma_issue(const DmaCtx& c, int k0, RAW& raw, WT& wt) {
#pragma unroll
  for (int j = 0; j < 4; ++j) dma16(c.xsrc[j] + size_t(k0) * 8, &raw[(2 * (4 * c.wave + j)) * kRawRow]);
#pragma unroll
  for (int j = 0; j < CB; ++j) dma16(c.wsrc[j] + k0, &wt[(16 * (CB * c.wave + j)) * kBK]);
}

// Three stages: step s computes on stage s % 3 while the DMAs of steps s + 1
// (issued one step earlier) and s + 2 (issued here, into the stage step s - 1
// read) are in flight.
template <int CB, class RAW, class WT, class RAWN, class WTN>
__device__ __forceinline__ void dma_step(const DmaCtx& c, bool ahead, bool next, int k_next, const RAW& raw,
                                         const WT& wt, RAWN& raw_n, WTN& wt_n, int (&colsum)[CB],
                                         v16i (&acc)[4][CB]) {
  // this wave's DMAs for this step are done: loads complete in order, and
  // `ahead` says whether the next step's 4 + CB are still allowed in flight;
  // after the barrier every wave's are, and every wave has finished reading
  // the stage the new DMAs overwrite
  if (ahead) {
    if (CB == 2)
      asm volatile("s_waitcnt vmcnt(6)\n\ts_barrier" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(7)\n\ts_barrier" ::: "memory");
  } else {
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  }
  if (next) dma_issue<CB>(c, k_next, raw_n, wt_n);
  // ---- every operand of the step first (16 transpose reads, 2 CB weight
  // reads), so that the MFMAs then issue back to back behind one LDS wait
  v4i aop[kBK / 32][4], bop[kBK / 32][CB];
#pragma unroll
  for (int ks = 0; ks < kBK / 32; ++ks) {
    const int chunk = ks * 2 + c.khalf;  // logical 16-byte chunk of the weight rows
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      const int row = c.wn * 32 * CB + cb * 32 + c.i;
      bop[ks][cb] = *reinterpret_cast<const v4i*>(&wt[row * kBK + ((chunk ^ wt_swizzle(row)) * 16)]);
    }
    const int k = ks * 32 + c.tr_k;
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const int r = c.wm * 16 + rb * 4 + c.tr_row;
      const v2i lo = tr8(raw, raw_offset(r, k)), hi = tr8(raw, raw_offset(r, k + 8));
      aop[ks][rb] = v4i{lo.x, lo.y, hi.x, hi.y};
    }
  }
  // ---- MFMA over the two 32-wide K steps
#pragma unroll
  for (int ks = 0; ks < kBK / 32; ++ks) {
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      // offset-binary digits: a_d = b_d - 128
      const v4i a = aop[ks][rb] ^ int(0x80808080u);
#pragma unroll
      for (int cb = 0; cb < CB; ++cb)
        acc[rb][cb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bop[ks][cb], acc[rb][cb], 0, 0, 0);
    }
  }
  // ---- column sums from the weight operands already in registers (lanes l
  // and l ^ 32 hold the two halves of each row's K chunk; VALU work beside
  // the MFMAs)
#pragma unroll
  for (int ks = 0; ks < kBK / 32; ++ks)
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
      for (int e = 0; e < 4; ++e) colsum[cb] = __builtin_amdgcn_sdot4(bop[ks][cb][e], 0x01010101, colsum[cb], false);
}

// Software-pipelined form (CB = 3, one wave per SIMD): each step runs as two
// halves of one 32-wide K step each, and the operands of the next half are
// read from LDS while the MFMAs of the current half run, so LDS reads and the
// matrix cores overlap within the wave with two operand sets in registers.
template <int CB>
struct HalfOps {
  v4i a[4], b[CB];
};

template <int CB, int KS, class RAW, class WT>
__device__ __forceinline__ void read_half(const DmaCtx& c, const RAW& raw, const WT& wt, HalfOps<CB>& o) {
  constexpr int ks = KS;
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) o.b[cb] = *reinterpret_cast<const v4i*>(&wt[c.w_off[ks] + 2048 * cb]);
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    const int blk = 2048 * rb + 256 * (ks ^ (rb & 1));
    const v2i lo = tr8(raw, c.a_off[0] + blk), hi = tr8(raw, c.a_off[1] + blk);
    o.a[rb] = v4i{lo.x, lo.y, hi.x, hi.y};
  }
}

template <int CB>
__device__ __forceinline__ void mfma_half(HalfOps<CB>& o, int (&colsum)[CB], v16i (&acc)[4][CB]) {
  // offset-binary digits, in place, all four before the first MFMA (a VALU
  // write just before the MFMA that reads it stalls the issue)
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) o.a[rb] ^= int(0x80808080u);
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
      acc[rb][cb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.a[rb], o.b[cb], acc[rb][cb], 0, 0, 0);
  }
  // column sums from the weight operands (lanes l and l ^ 32 hold the two
  // halves of each row's K chunk)
#pragma unroll
  for (int cb = 0; cb < CB; ++cb)
#pragma unroll
    for (int e = 0; e < 4; ++e) colsum[cb] = __builtin_amdgcn_sdot4(o.b[cb][e], 0x01010101, colsum[cb], false);
}

// 3 + 8 LDS reads among the 4 CB MFMAs of a half.
template <int CB>
__device__ __forceinline__ void interleave_half() {
  __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // the four digit XORs
#pragma unroll
  for (int j = 0; j < CB + 8; ++j) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
  }
}

// Step s: half A reads K step 1 of stage s (raw_s, wt_s) into h1 while the
// MFMAs of K step 0 run from h0; then the wait for step s + 1's stage and the
// refill of stage s with step s + 3 (past the last step: the last step's tile
// again, never read); half B reads K step 0 of stage s + 1 (raw_n, wt_n; past
// the last step: stale data, never used) into h0 while the MFMAs of K step 1
// run from h1.
template <int CB, class RAWS, class WTS, class RAWN, class WTN>
__device__ __forceinline__ void piped_step(const DmaCtx& c, int s, int steps, int k_begin, RAWS raw_s, WTS wt_s,
                                           RAWN raw_n, WTN wt_n, HalfOps<CB>& h0, HalfOps<CB>& h1,
                                           int (&colsum)[CB], v16i (&acc)[4][CB]) {
  read_half<CB, 1>(c, raw_s, wt_s, h1);
  mfma_half<CB>(h0, colsum, acc);
  interleave_half<CB>();
  // step s + 1's DMAs are done when only step s + 2's (4 + CB = 7) remain in
  // flight, and this wave's reads of stage s are done; after the barrier both
  // hold for every wave, so stage s may be refilled
  asm volatile("s_waitcnt vmcnt(7) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  dma_issue<CB>(c, k_begin + min(s + 3, steps - 1) * kBK, raw_s, wt_s);
  read_half<CB, 0>(c, raw_n, wt_n, h0);
  mfma_half<CB>(h1, colsum, acc);
  interleave_half<CB>();
}

// a m + c for signed 32-bit a, m and a 64-bit c, as one v_mad_i64_i32 (the
// compiler expands a product by a power of two into a sign extension and
// 64-bit shifts and adds, several instructions per term).  Its carry-out
// lane mask is not read.
__device__ __forceinline__ int64_t mad_i64(int a, int m, int64_t c) {
  int64_t r;
  uint64_t unused;
  asm("v_mad_i64_i32 %0, %1, %2, %3, %4" : "=v"(r), "=s"(unused) : "v"(a), "s"(m), "v"(c));
  return r;
}

// Tile (tm, tn) of this workgroup in the gridDim.y x gridDim.x tile grid.
// Workgroups go to the 8 XCDs round robin (linear id mod 8), so when the grid
// holds a multiple of 8 tiles XCD x is given the contiguous range
// [x nt/8, (x+1) nt/8) of a grouped order (8 tile rows at a time, column by
// column within the group): a compact block of tiles whose share rows and
// weight columns stay in that XCD's L2 (512 x 3072 in 32 x 192 tiles: each
// XCD 8 x 4 tiles, 2 MiB of shares and 768 KiB of weights).  Any bijection
// is correct; this one only places the reuse.
__device__ __forceinline__ void tile_of(int& tm, int& tn) {
  const int TN = int(gridDim.x), TM = int(gridDim.y), nt = TN * TM;
  int t = int(blockIdx.y) * TN + int(blockIdx.x);
  if (nt % 8 == 0) t = (t % 8) * (nt / 8) + t / 8;
  constexpr int G = 8;
  const int group = t / (G * TN), first = group * G, rows = min(G, TM - first);
  const int in = t - group * G * TN;
  tm = first + in % rows;
  tn = in / rows;
}

// Epilogue of one accumulator tile of a wave: rows row0 .. row0 + 3 (this lane
// writes rows row0 + 2 khalf and row0 + 2 khalf + 1), column col.  The lane
// holds, for its column, digits 4 khalf .. 4 khalf + 3 of the four rows in
// register groups g (rows row0 + g); the halves of the wave add their digit
// sums with v_permlane32_swap: swapping lanes 32-63 of part[g] with lanes 0-31
// of part[g + 2] leaves every lane with its own half's value and the other
// half's for the row it writes, one in each register.  corr is the
// offset-binary correction of the column, sh its shift.
__device__ __forceinline__ void store_tile(const v16i& a, int row0, int col, int khalf, uint64_t corr, int sh,
                                           bool split, uint64_t mask, uint64_t* __restrict__ y, int M, int N) {
  uint64_t part[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    // sum_ii acc_ii 256^ii fits 56 signed bits: three 32x32+64 MADs
    const int64_t v = mad_i64(a[4 * g + 3], 16777216, mad_i64(a[4 * g + 2], 65536, mad_i64(a[4 * g + 1], 256, int64_t(a[4 * g]))));
    part[g] = uint64_t(v) << (32 * khalf);
  }
  uint64_t sum[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const auto lo = __builtin_amdgcn_permlane32_swap(uint32_t(part[h]), uint32_t(part[h + 2]), false, false);
    const auto hi = __builtin_amdgcn_permlane32_swap(uint32_t(part[h] >> 32), uint32_t(part[h + 2] >> 32), false, false);
    sum[h] = ((uint64_t(hi[0]) << 32) | lo[0]) + ((uint64_t(hi[1]) << 32) | lo[1]);
  }
  if (col >= N) return;  // the same for lanes l and l ^ 32
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int row = row0 + 2 * khalf + h;
    if (row >= M) continue;
    uint64_t v = corr + sum[h];
    v = sh < 64 ? (v << sh) : 0;
    if (split)
      atomicAdd(reinterpret_cast<unsigned long long*>(y + size_t(row) * N + col), (unsigned long long)v);
    else
      y[size_t(row) * N + col] = v & mask;
  }
}

// The offset-binary correction 0x8080808080808080 sum_k w[col][k] of a column
// from this lane's column sum (lanes l and l ^ 32 hold the two halves of the
// column's K chunks; after the swap one register holds lanes 0-31's values in
// both halves, the other lanes 32-63's).
__device__ __forceinline__ uint64_t column_correction(int colsum) {
  const auto cs = __builtin_amdgcn_permlane32_swap(colsum, colsum, false, false);
  return 0x8080808080808080ull * uint64_t(int64_t(int(cs[0])) + int64_t(int(cs[1])));
}

// Weight planes: w holds `planes` int8 matrices [planes][N][K], plane e the
// signed byte of weight digit e (planes = 1: int8 weights; 3: the pre-split
// f12 weights).  Workgroup z takes plane z / splits and K split z % splits;
// plane e's products enter y shifted by 8e.  CB = 2: 128-column tiles, two
// workgroups (two waves per SIMD) per CU, whose waits overlap; CB = 3:
// 192-column tiles, one workgroup per CU, 12 accumulator tiles per wave, so
// that every MFMA takes fewer operand bytes from L2 and LDS.
template <int CB>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(CB == 2 ? 2 : 1, CB == 2 ? 2 : 1)))
    share_gemm_dma_kernel(const uint64_t* __restrict__ x, const int8_t* __restrict__ w,
                          const int8_t* __restrict__ shifts, uint64_t* __restrict__ y, int M, int K, int N,
                          uint64_t mask, int k_split, int splits) {
  constexpr int BN = 64 * CB;
  const int plane = int(blockIdx.z) / splits, split_z = int(blockIdx.z) % splits;
  w += size_t(plane) * size_t(N) * size_t(K);
  __shared__ __attribute__((aligned(16))) uint8_t raw0[kBM * kRawRow];
  __shared__ __attribute__((aligned(16))) uint8_t raw1[kBM * kRawRow];
  __shared__ __attribute__((aligned(16))) uint8_t raw2[kBM * kRawRow];
  __shared__ __attribute__((aligned(16))) uint8_t wt0[BN * kBK];
  __shared__ __attribute__((aligned(16))) uint8_t wt1[BN * kBK];
  __shared__ __attribute__((aligned(16))) uint8_t wt2[BN * kBK];

  const int t = threadIdx.x, lane = t & 63;
  DmaCtx c;
  c.wave = t >> 6;
  c.wm = c.wave >> 1;
  c.wn = c.wave & 1;
  c.i = lane & 31;
  c.khalf = lane >> 5;
  // transpose-read source of this lane: share row 2((l/16) % 2) + l % 2 of
  // the 4-row block, word (l/2) % 8 of the 8-word run at k = 16(l/32)
  c.tr_row = 2 * ((lane >> 4) & 1) + (lane & 1);
  c.tr_k = 16 * (lane >> 5) + ((lane >> 1) & 7);
  {
    const int j = (lane >> 1) & 7;
#pragma unroll
    for (int h = 0; h < 2; ++h)
      c.a_off[h] = (c.wm * 16 + c.tr_row) * kRawRow + 16 * (((8 * c.khalf + 4 * h) ^ (4 * c.tr_row)) + (j >> 1)) +
                   8 * (j & 1);
    const int f = wt_swizzle(c.i);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      c.w_off[ks] = (c.wn * 32 * CB + c.i) * kBK + 16 * (2 * (ks ^ (f >> 1)) + (c.khalf ^ (f & 1)));
  }
  int tm, tn;
  tile_of(tm, tn);
  const int m0 = tm * kBM, n0 = tn * BN;
  // DMA sources of this lane: 4 raw-share instructions (2 rows of 512 B each)
  // and CB weight instructions (16 rows of 64 B each) per wave and step.
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = 2 * (4 * c.wave + j) + (lane >> 5);
    const int grow = min(m0 + row, M - 1);  // rows past M: any valid row, results dropped
    const int ck = (lane & 31) ^ (4 * (row & 7));  // logical chunk stored at physical chunk lane & 31
    c.xsrc[j] = reinterpret_cast<const uint8_t*>(x + size_t(grow) * K) + ck * 16;
  }
#pragma unroll
  for (int j = 0; j < CB; ++j) {
    const int row = 16 * (CB * c.wave + j) + (lane >> 2);
    const int grow = min(n0 + row, N - 1);
    const int ck = (lane & 3) ^ wt_swizzle(row);  // logical chunk stored at physical chunk lane & 3
    c.wsrc[j] = w + size_t(grow) * K + ck * 16;
  }
  int colsum[CB];
  v16i acc[4][CB];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    colsum[cb] = 0;
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) acc[rb][cb] = v16i{0};
  }

  // split-K: workgroup z takes K steps [z k_split, (z+1) k_split); with more
  // than one split the partial products are added into y (zeroed first) by
  // 64-bit atomics, exact mod 2^64 in any order
  const int k_begin = split_z * k_split;
  const int steps = min(k_split, K - k_begin) / kBK;
  if constexpr (CB == 3) {
    auto raw_of = [&](int q) { return q == 0 ? raw0 : (q == 1 ? raw1 : raw2); };
    auto wt_of = [&](int q) { return q == 0 ? wt0 : (q == 1 ? wt1 : wt2); };
    // steps 0..2 in flight (past the last step: the last step's tile again)
    dma_issue<CB>(c, k_begin, raw0, wt0);
    dma_issue<CB>(c, k_begin + min(1, steps - 1) * kBK, raw1, wt1);
    dma_issue<CB>(c, k_begin + min(2, steps - 1) * kBK, raw2, wt2);
    asm volatile("s_waitcnt vmcnt(14)\n\ts_barrier" ::: "memory");
    HalfOps<CB> h0, h1;
    read_half<CB, 0>(c, raw0, wt0, h0);
    int q = 0;  // stage of step s
    for (int s = 0; s < steps; ++s) {
      const int qn = q == 2 ? 0 : q + 1;
      piped_step<CB>(c, s, steps, k_begin, raw_of(q), wt_of(q), raw_of(qn), wt_of(qn), h0, h1, colsum, acc);
      q = qn;
    }
    // the refills past the last step land before the workgroup ends
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  } else {
  dma_issue<CB>(c, k_begin, raw0, wt0);
  if (steps > 1) dma_issue<CB>(c, k_begin + kBK, raw1, wt1);
  for (int s = 0; s < steps; s += 3) {
    const int kn = k_begin + (s + 2) * kBK;
    dma_step<CB>(c, s + 1 < steps, s + 2 < steps, kn, raw0, wt0, raw2, wt2, colsum, acc);
    if (s + 1 < steps) dma_step<CB>(c, s + 2 < steps, s + 3 < steps, kn + kBK, raw1, wt1, raw0, wt0, colsum, acc);
    if (s + 2 < steps) dma_step<CB>(c, s + 3 < steps, s + 4 < steps, kn + 2 * kBK, raw2, wt2, raw1, wt1, colsum, acc);
  }
  }
  const bool split = gridDim.z > 1;

  // ---- epilogue: column sums, digit recombination, shift, mask
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    const int col = n0 + c.wn * 32 * CB + cb * 32 + c.i;
    const uint64_t corr = column_correction(colsum[cb]);
    const int sh = 8 * plane + (shifts && col < N ? int(shifts[col]) : 0);
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
      store_tile(acc[rb][cb], m0 + c.wm * 16 + rb * 4, col, c.khalf, corr, sh, split, mask, y, M, N);
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

// Zero several outputs in one launch (a batch's split-K products): blockIdx.y
// names the buffer.
__global__ void __launch_bounds__(256) gemm_clear_list_kernel(GemmClearList l) {
  uint64_t* y = l.ptr[blockIdx.y];
  const size_t n = l.words[blockIdx.y];
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x) y[i] = 0;
}

hipError_t launch_gemm_clear_list(const GemmClearList& l, hipStream_t s) {
  if (l.count <= 0) return hipSuccess;
  hipLaunchKernelGGL(gemm_clear_list_kernel, dim3(512, unsigned(l.count)), dim3(256), 0, s, l);
  return hipGetLastError();
}

// Split-K products add their partial products into y with atomics, so y must
// be zero first; true when this product takes that path.
bool share_gemm_adds_into_y(const void* x, const void* w, int w_bits, int M, int K, int N) {
  if (w_bits != 8 && w_bits != 24) return false;
  const int w_vec = (K % 16 == 0) && (reinterpret_cast<uintptr_t>(w) % 16 == 0);
  if (!(K % kBK == 0 && w_vec && reinterpret_cast<uintptr_t>(x) % 16 == 0)) return false;
  const int planes = w_bits == 8 ? 1 : 3, ksteps = K / kBK;
  const long tiles2 = long((N + 127) / 128) * long((M + kBM - 1) / kBM);
  int splits = 1;
  while (splits < 4 && tiles2 * splits < 256 && ksteps / (splits * 2) >= 8) splits *= 2;
  const int k_split = (ksteps + splits - 1) / splits * kBK;
  return ((K + k_split - 1) / k_split) * planes > 1;
}

hipError_t launch_share_gemm(const uint64_t* x, const void* w, int w_bits, const int8_t* shifts, uint64_t* y,
                             int M, int K, int N, int mask_bits, hipStream_t s, bool y_zero) {
  const uint64_t mask = mask_bits >= 64 ? ~0ull : ((1ull << mask_bits) - 1);
  const dim3 grid((N + kBN - 1) / kBN, (M + kBM - 1) / kBM), block(kThreads);
  // 16-byte weight loads need 16-byte aligned rows
  const int w_vec = (K % 16 == 0) && (reinterpret_cast<uintptr_t>(w) % 16 == 0);
  if (w_bits == 8 || w_bits == 24) {
    const int planes = w_bits == 8 ? 1 : 3;
    if (K % kBK == 0 && w_vec && reinterpret_cast<uintptr_t>(x) % 16 == 0) {
      // 128-column tiles (CB = 2, up to two workgroups per CU), K split while
      // the tiles fill fewer than 256 workgroups and each split keeps >= 8
      // steps.  192-column tiles (CB = 3, one workgroup per CU) only where
      // they fill the 256 CUs in one round while the 128-column grid would
      // leave the CUs unevenly loaded (between one and two workgroups each):
      // 512 x 1024 x 3072 int8 runs 21.4 us against 22.8 us; every other
      // Qwen3 shape and the f12 planes run faster with CB = 2 (measured).
      const int ksteps = K / kBK;
      const long tiles2 = long((N + 127) / 128) * long((M + kBM - 1) / kBM);
      const long tiles3 = long((N + 191) / 192) * long((M + kBM - 1) / kBM);
      int best_splits = 1;
      while (best_splits < 4 && tiles2 * best_splits < 256 && ksteps / (best_splits * 2) >= 8) best_splits *= 2;
      const long wg2 = tiles2 * best_splits * planes;
      const int best_cb = (best_splits == 1 && planes == 1 && wg2 > 256 && wg2 < 512 && tiles3 <= 256) ? 3 : 2;
      const int k_split = (ksteps + best_splits - 1) / best_splits * kBK;
      const int splits = (K + k_split - 1) / k_split;
      const size_t words = size_t(M) * N;
      const unsigned fgrid = unsigned(std::min<size_t>((words + 255) / 256, 4096));
      // several planes or K splits add their partial products into y
      const bool atomic = splits * planes > 1;
      if (atomic && !y_zero) {
        hipLaunchKernelGGL(gemm_clear_kernel, dim3(fgrid), dim3(256), 0, s, y, words, 0ull);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
      }
      const unsigned gy = unsigned((M + kBM - 1) / kBM), gz = unsigned(splits * planes);
      if (best_cb == 2)
        hipLaunchKernelGGL(share_gemm_dma_kernel<2>, dim3(unsigned((N + 127) / 128), gy, gz), block, 0, s, x,
                           static_cast<const int8_t*>(w), shifts, y, M, K, N, mask, k_split, splits);
      else
        hipLaunchKernelGGL(share_gemm_dma_kernel<3>, dim3(unsigned((N + 191) / 192), gy, gz), block, 0, s, x,
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
