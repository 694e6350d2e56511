// wt_gemm.hip — C = A^T B in float32 from float32 operands on the bf16 matrix cores.
//
// The rate networks' weight gradient dL/dW = sum over (trial, step) of presynaptic rates
// times dL/da (rate/engine.py:365-377, a float32 matrix product in the reference) has a
// long contraction (K = trials x steps, 256,000 at configuration 4) over two float32
// operands stored k-major: A (K x M), B (K x N), C (M x N), all row-major.
//
// Each operand element x is split in registers into bfloat16 hi = bf16(x) and lo =
// bf16(x - hi) (round to nearest even; x = hi + lo to 2^-18 relative), and the product
// is hi.hi + hi.lo + lo.hi on v_mfma_f32_32x32x16_bf16, accumulated in float32: each term
// within 3 * 2^-18 of its float32 value (the lo.lo term, below 2^-18, is dropped).
//
// Tiles: 256 x 256 outputs per workgroup of 8 waves (4 along M x 2 along N; a wave owns
// 64 x 128 = 2 x 4 blocks of 32 x 32). K runs in stages of 32: every thread loads 16
// elements of A and 16 of B (8 consecutive k of one column, twice: each load instruction
// reads one k row, 64 consecutive columns across the wave), splits them and stores each
// group of 8 k as one 16-byte bf16 chunk — the MFMA operand layout, k contiguous per row
// (M row of A, N row of B) — into two LDS buffers (stage s + 1 is loaded into registers
// while stage s multiplies). Rows are 64 bytes (4 chunks); chunk c of row r sits in slot
// c ^ ((r / 4) % 4), so the 16 lanes of an operand read (rows r .. r + 15, one chunk)
// cover all 64 banks.
//
// Workgroups are mapped to tiles so that the 32 workgroups on one XCD (workgroup i runs
// on XCD i % 8) share operand columns in that XCD's L2: with 16 x 16 tiles, XCD x takes
// tile rows 4 (x / 2) .. + 3 and tile columns 8 (x % 2) .. + 7.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/wiretorch_amd.h"

namespace wt {
namespace gemm {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;

constexpr int kTile = 256;     // outputs per workgroup, per side
constexpr int kStageK = 32;    // k per stage
constexpr int kThreads = 512;  // 8 waves
constexpr int kChunks = kStageK / 8;  // 16-byte chunks per LDS row

// One operand piece of a stage in LDS: [256 rows][4 chunks] of 8 bf16.
typedef uint4 Piece[kTile * kChunks];
struct Stage {
  Piece a_hi, a_lo, b_hi, b_lo;  // 64 KB
};

__device__ inline int slot(int row, int chunk) { return row * kChunks + (chunk ^ ((row >> 2) & 3)); }

__device__ inline float gload(const float* p) {
  return *(const __attribute__((address_space(1))) float*)p;
}

// A thread's share of one operand's stage: column `col` of the tile, k groups g and g + 2
// (8 k each), loaded as 16 scalars. Each load instruction of a wave reads 64 consecutive
// columns of one k row (two whole 128-byte lines).
struct Regs {
  float v[2][8];
};

// Loads go through a buffer resource whose base is the stage's first row (k0) and whose
// range ends at row K: a row past K reads zero with no check. A thread's element (row kr,
// column c) is at byte offset (kr * ld + c) * 4, all of it in the lane's offset register
// (the range check covers that offset, not the scalar one). A column past the operand's
// width (a partial tile) gets an offset past the range: it reads zero too.
constexpr uint32_t kRsrcWord3 = 0x00020000;  // raw buffer access (GFX9 family)

__device__ inline void load_stage(Regs& r, const float* X, uint32_t ld, int64_t K,
                                  int64_t ncols, int64_t k0, int64_t c0, int col, int g) {
  const int64_t left = (K - k0) * (int64_t)ld * 4;  // bytes from row k0 to row K
  const uint32_t range = left > 0x7fffffff ? 0x7fffffffu : (uint32_t)(left > 0 ? left : 0);
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(X + k0 * (int64_t)ld), (short)0, (int)range, (int)kRsrcWord3);
  const bool in_col = c0 + col < ncols;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t voff = in_col ? ((uint32_t)(8 * (g + 2 * h)) * ld + (uint32_t)(c0 + col)) * 4u
                                 : 0x80000000u;
#pragma unroll
    for (int e = 0; e < 8; ++e)
      r.v[h][e] = __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(rsrc, (int)(voff + e * ld * 4u), 0, 0));
  }
}

// Each group of 8 k split into bf16 hi and lo, stored as one 16-byte chunk each: chunk
// g + 2 h of LDS row `col`.
__device__ inline void split_store(const Regs& r, Piece& hi, Piece& lo, int col, int g) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    bf16x8 H, L;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const __bf16 x = (__bf16)r.v[h][e];  // round to nearest even
      H[e] = x;
      L[e] = (__bf16)(r.v[h][e] - (float)x);
    }
    const int s = slot(col, g + 2 * h);
    hi[s] = *reinterpret_cast<const uint4*>(&H);
    lo[s] = *reinterpret_cast<const uint4*>(&L);
  }
}

__device__ inline bf16x8 frag(const Piece& p, int row, int chunk) {
  const uint4 u = p[slot(row, chunk)];
  return *reinterpret_cast<const bf16x8*>(&u);
}

// Output element v of a lane's 32 x 32 block: row 8(v/4) + 4(l/32) + v%4, column l%32.
__device__ inline int out_row(int v, int lane) { return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3); }

__global__ __launch_bounds__(kThreads) void gemm_tn_split_kernel(
    const float* __restrict__ A, uint32_t lda, const float* __restrict__ B, uint32_t ldb,
    float* __restrict__ C, int64_t ldc, int64_t K, int64_t M, int64_t N, int32_t accumulate,
    int32_t tiles_m, int32_t tiles_n) {
  extern __shared__ __align__(16) unsigned char smem[];
  Stage* st = reinterpret_cast<Stage*>(smem);  // two stages
  // XCD-aware tile of this workgroup
  const int wg = blockIdx.x;
  int ti, tj;
  if (tiles_m == 16 && tiles_n == 16) {
    const int x = wg & 7, local = wg >> 3;  // 32 tiles per XCD
    ti = (x >> 1) * 4 + (local >> 3);
    tj = (x & 1) * 8 + (local & 7);
  } else {
    ti = wg / tiles_n;
    tj = wg - ti * tiles_n;
  }
  const int64_t m0 = (int64_t)ti * kTile, n0 = (int64_t)tj * kTile;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int col = tid & 255, g = tid >> 8;  // loader: column, first k group
  const int wm = wave & 3, wn = wave >> 2;  // the wave's 64 x 128 sub-tile
  f32x16 acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

  const int64_t stages = (K + kStageK - 1) / kStageK;
  Regs ra, rb;
  load_stage(ra, A, lda, K, M, 0, m0, col, g);
  load_stage(rb, B, ldb, K, N, 0, n0, col, g);
  split_store(ra, st[0].a_hi, st[0].a_lo, col, g);
  split_store(rb, st[0].b_hi, st[0].b_lo, col, g);
  __syncthreads();
  auto products = [&](const Stage& S, int kk) {
    const int chunk = 2 * kk + (lane >> 5);
    bf16x8 ah[2], al[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int row = wm * 64 + i * 32 + (lane & 31);
      ah[i] = frag(S.a_hi, row, chunk);
      al[i] = frag(S.a_lo, row, chunk);
    }
    // B fragments one block at a time (their registers reused): 6 MFMAs per pair read
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = wn * 128 + j * 32 + (lane & 31);
      const bf16x8 bh = frag(S.b_hi, row, chunk), bl = frag(S.b_lo, row, chunk);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i], bh, acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i], bl, acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[i], bh, acc[i][j], 0, 0, 0);
      }
    }
  };
  // Per stage: the next stage's loads are issued first (past the last stage they read the
  // range's end: zeros, stored into the buffer nobody reads again); the first half of the
  // stage's products; the next stage's split and stores into the other buffer (last read
  // before the previous barrier), between the two halves, so that the matrix cores run
  // one wave's products while the other wave splits; the second half; one barrier.
  for (int64_t s = 0; s < stages; ++s) {
    const int cur = (int)(s & 1);
    load_stage(ra, A, lda, K, M, (s + 1) * kStageK, m0, col, g);
    load_stage(rb, B, ldb, K, N, (s + 1) * kStageK, n0, col, g);
    const Stage& S = st[cur];
    products(S, 0);
    Stage& nxt = st[cur ^ 1];
    split_store(ra, nxt.a_hi, nxt.a_lo, col, g);
    split_store(rb, nxt.b_hi, nxt.b_lo, col, g);
    products(S, 1);
    __syncthreads();
  }
  // C block (i, j) of the wave: rows m0 + wm 64 + 32 i + out_row, column n0 + wn 128 + 32 j + l % 32
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t n = n0 + wn * 128 + j * 32 + (lane & 31);
      if (n >= N) continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t m = m0 + wm * 64 + i * 32 + out_row(v, lane);
        if (m >= M) continue;
        float* c = C + m * ldc + n;
        *c = accumulate ? *c + acc[i][j][v] : acc[i][j][v];
      }
    }
}

}  // namespace gemm
}  // namespace wt

extern "C" int wt_gemm_tn_split(const float* A, int64_t lda, const float* B, int64_t ldb,
                                float* C, int64_t ldc, int64_t K, int64_t M, int64_t N,
                                int32_t accumulate, wt_stream_t stream) {
  using namespace wt::gemm;
  if (K < 0 || M < 0 || N < 0 || lda < M || ldb < N || ldc < N) return hipErrorInvalidValue;
  // byte offsets within a stage (32 rows of the widest operand) are formed in 32 bits
  if (lda * kStageK * 4 >= INT32_MAX || ldb * kStageK * 4 >= INT32_MAX) return hipErrorInvalidValue;
  if (M == 0 || N == 0) return hipSuccess;
  if (!A || !B || !C) return hipErrorInvalidValue;
  const int64_t tm = (M + kTile - 1) / kTile, tn = (N + kTile - 1) / kTile;
  if (tm * tn > INT32_MAX) return hipErrorInvalidValue;
  const size_t lds = 2 * sizeof(Stage);
  const void* fn = reinterpret_cast<const void*>(&gemm_tn_split_kernel);
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(gemm_tn_split_kernel, dim3((unsigned)(tm * tn)), dim3(kThreads), lds,
                     (hipStream_t)stream, A, (uint32_t)lda, B, (uint32_t)ldb, C, ldc, K, M, N, accumulate,
                     (int32_t)tm, (int32_t)tn);
  return hipGetLastError();
}
