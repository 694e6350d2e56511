// wt_rate.hip — rate networks on gfx950: the step of rate/dynamics.py as one fused launch
// per step (an MFMA matrix product of the rates with the weights, whose epilogue filters
// the currents, integrates the voltages and outputs the next rates), and its reverse.
//
// Every matrix operand is zero-padded to whole tiles by the host, so the tile loads need
// no bounds checks:
//   * the forward product's K dimension holds every pathway's rows as a segment of whole
//     k-blocks (recurrent pathways first: their rows are neurons, read from the rate
//     buffer `rin`; then the feedforward pathways: their rows are input columns, read
//     from the padded input X of the step); W is (K_pad x N_pad);
//   * a segment's partial product is the pathway's activation a_k; at the end of the
//     segment it enters the synaptic targets, target[s] += a_k * scale_k * made_k[s], in
//     pathway order as the reference sums them.
// Tiles: 64 x 64 outputs per workgroup of four waves; stages of 128 bytes of k staged
// in LDS, each wave multiplying the whole tile over a quarter of every stage, the four
// partials added in wave order at the end of each pathway's segment. MFMA:
// v_mfma_f32_32x32x2_f32 (float32 storage) or v_mfma_f32_32x32x16_bf16 (bfloat16
// storage), accumulating in float32.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/wiretorch_amd.h"

namespace wt {
namespace rate {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kTile = 64;     // outputs per workgroup, per side
constexpr int kMaxSlices = 4; // k slices of the forward's split product
constexpr int kThreads = 256;
constexpr int kMaxS = 8;
constexpr int kMaxSeg = 16;

// The reference's nonlinearities (rate/dynamics.py:63-69, torch's definitions) and
// their derivatives. Codes follow wiretorch_amd.rate.NONLINEARITIES.
__device__ inline float nonlin(int code, float x) {
  switch (code) {
    case 0: return x > 0.0f ? x : 0.0f;                        // relu
    case 1: return x > 20.0f ? x : log1pf(expf(x));            // softplus (beta 1, threshold 20)
    case 2: return 1.0f / (1.0f + expf(-x));                   // sigmoid
    default: return tanhf(x);                                  // tanh
  }
}
// The same for M values of one neuron (one code): the switch is taken once, so that the
// M evaluations are independent and interleave.
template <int M>
__device__ inline void nonlin_n(int code, float gain, const float (&x)[M], float (&r)[M]) {
  switch (code) {
    case 0:
#pragma unroll
      for (int v = 0; v < M; ++v) r[v] = gain * (x[v] > 0.0f ? x[v] : 0.0f);
      break;
    case 1:
#pragma unroll
      for (int v = 0; v < M; ++v) r[v] = gain * (x[v] > 20.0f ? x[v] : log1pf(expf(x[v])));
      break;
    case 2:
#pragma unroll
      for (int v = 0; v < M; ++v) r[v] = gain * (1.0f / (1.0f + expf(-x[v])));
      break;
    default:
#pragma unroll
      for (int v = 0; v < M; ++v) r[v] = gain * tanhf(x[v]);
      break;
  }
}
__device__ inline float nonlin_grad(int code, float x) {
  switch (code) {
    case 0: return x > 0.0f ? 1.0f : 0.0f;
    case 1: {
      if (x > 20.0f) return 1.0f;
      const float z = expf(x);
      return z / (z + 1.0f);
    }
    case 2: {
      const float s = 1.0f / (1.0f + expf(-x));
      return s * (1.0f - s);
    }
    default: {
      const float t = tanhf(x);
      return 1.0f - t * t;
    }
  }
}

// Output element v of a lane's 32 x 32 block: row 8(v/4) + 4(l/32) + v%4, column l%32.
__device__ inline int out_row(int v, int lane) { return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3); }

// ---------------------------------------------------------------------------------
// The tile product C[64 x 64] += A[64 x k] Bt[64 x k]^T with both operands k-contiguous
// (row-major, k along the row: the rates or inputs by trial, the weights transposed by
// target), in stages of 128 bytes of k (64 bfloat16 or 32 float32).
//
// A stage is 8 KB per operand: thread t fetches the 16-byte chunk t % 8 of rows t / 8 and
// 32 + t / 8, so eight consecutive threads read one row's 128 bytes. Stages are fetched
// kDepth ahead into a ring of registers and stored to LDS. In LDS, chunk c of row r sits
// in slot c ^ sw(r) of its row, sw(r) = (r % 8) ^ ((r / 8) % 2): an MFMA operand read
// (one 16-byte chunk per lane, one chunk of rows r..r+15 per 16 lanes) then covers all
// 64 banks (256 bytes: row parity selects the half, the slot the 16 bytes) — and with
// 32 banks, each 8 lanes' rows fall in 8 different slots — no bank conflicts.
// ---------------------------------------------------------------------------------

constexpr int kStageBytes = 128;
constexpr int kDepth = 4;

struct StageRegs {
  u32x4 a[2], b[2];
};

__device__ inline u32x4 gload16(const char* p) {
  return *(const __attribute__((address_space(1))) u32x4*)p;
}

// One stage's operands: rows [0, 64) of A at byte offset `a` (row pitch lda bytes), of
// Bt at `b` (pitch ldb).
__device__ inline void stage_load(StageRegs& r, const char* a, int64_t lda, const char* b,
                                  int64_t ldb) {
  const int t = threadIdx.x, row = t >> 3, off = (t & 7) * 16;
  r.a[0] = gload16(a + row * lda + off);
  r.a[1] = gload16(a + (row + 32) * lda + off);
  r.b[0] = gload16(b + row * ldb + off);
  r.b[1] = gload16(b + (row + 32) * ldb + off);
}

// LDS: [buffer][operand][row * 8 + slot] in 16-byte units; three buffers.
constexpr int kBuffers = 3;
typedef u32x4 StageLds[kBuffers][2][512];

__device__ inline int swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

__device__ inline void stage_store(StageLds& lds, int buf, const StageRegs& r) {
  const int t = threadIdx.x, row = t >> 3, slot = (t & 7) ^ swz(row);  // swz(row + 32) == swz(row)
  lds[buf][0][row * 8 + slot] = r.a[0];
  lds[buf][0][(row + 32) * 8 + slot] = r.a[1];
  lds[buf][1][row * 8 + slot] = r.b[0];
  lds[buf][1][(row + 32) * 8 + slot] = r.b[1];
}

// Each of the four waves multiplies the whole 64 x 64 tile (2 x 2 blocks of 32 x 32)
// over its own quarter of every stage's k — chunks 2w and 2w + 1 (16 bytes each) for
// wave w — and keeps its partial sums; `reduce` adds the four partials of a block in
// wave order. Per stage a wave reads 4 chunks per lane from LDS (not 8, as a 32 x 32
// block over the whole stage would), which halves the LDS reads per flop.
typedef f32x16 Acc[2][2];

// A wave's operands of one stage: rows r and 32 + r of A and of Bt at its chunk.
struct Frag {
  u32x4 x[2], y[2];
};

__device__ inline Frag frag_load(const u32x4 (&buf)[2][512], int wave, int lane) {
  const int r = lane & 31, chunk = 2 * wave + (lane >> 5);
  const int slot = chunk ^ swz(r);
  Frag f;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    f.x[i] = buf[0][(32 * i + r) * 8 + slot];
    f.y[i] = buf[1][(32 * i + r) * 8 + slot];
  }
  return f;
}

template <typename T>
struct Mma;
// bfloat16, v_mfma_f32_32x32x16_bf16: C += A[32 x 16] B[16 x 32], lane l supplying
// A[l % 32][8 (l / 32) + e] and B[8 (l / 32) + e][l % 32], e < 8: the 16 k of the
// wave's two chunks.
template <>
struct Mma<__bf16> {
  __device__ static void stage(Acc& c, const Frag& f) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        c[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            *reinterpret_cast<const bf16x8*>(&f.x[i]), *reinterpret_cast<const bf16x8*>(&f.y[j]),
            c[i][j], 0, 0, 0);
  }
};
// float32, v_mfma_f32_32x32x2_f32: C += A[32 x 2] B[2 x 32], lane l supplying one element
// of k-slot l / 32: MFMA step e takes element e of chunk 2w + l / 32 — A and B lanes
// agree on it, so each of the wave's 8 k enters exactly once.
template <>
struct Mma<float> {
  __device__ static void stage(Acc& c, const Frag& f) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          c[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(f.x[i][e]),
                                                         __uint_as_float(f.y[j][e]), c[i][j], 0,
                                                         0, 0);
  }
};

// LDS for `reduce`: [block][wave][v / 4][lane] in 16-byte units (64 KB).
typedef u32x4 ReduceLds[4][4][4][64];

// The sum over the four waves (in wave order) of block (w / 2, w % 2) of the tile, for
// the wave w that owns it; every wave's partials are then zero. All four partials of a
// block pass through LDS. A workgroup barrier inside: every wave calls it at the same
// point.
__device__ inline f32x16 reduce(Acc& c, ReduceLds& red, int wave, int lane) {
#pragma unroll
  for (int blk = 0; blk < 4; ++blk) {
    const f32x16& p = c[blk >> 1][blk & 1];
#pragma unroll
    for (int q = 0; q < 4; ++q)
      red[blk][wave][q][lane] = u32x4{__float_as_uint(p[4 * q]), __float_as_uint(p[4 * q + 1]),
                                      __float_as_uint(p[4 * q + 2]), __float_as_uint(p[4 * q + 3])};
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) c[i][j] = f32x16{};
  __syncthreads();
  f32x16 sum = {};
#pragma unroll
  for (int w = 0; w < 4; ++w)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const u32x4 x = red[wave][w][q][lane];
#pragma unroll
      for (int e = 0; e < 4; ++e) sum[4 * q + e] = sum[4 * q + e] + __uint_as_float(x[e]);
    }
  return sum;
}

// Runs a tile's product over G segments of stages (count(g) >= 1 stages each; src(g, l,
// a, lda, b, ldb) names stage l of segment g), calling fold(g, c) with the partial sums
// after each segment (fold may reduce them).
//
// Pipeline: stage s + 2 is stored to LDS while the MFMAs of stage s run on operands read
// from LDS during stage s - 1, and stage s + 1's operands are read meanwhile (three LDS
// buffers, one barrier per stage); global loads run kDepth stages ahead of the store,
// across segment ends. Each segment runs a whole number of kDepth-stage trips with no
// exit inside: its stages past count(g) (at most kDepth - 1) load, store and synchronise
// like the others — fetching a real stage again — but multiply zeros. The loads in
// flight are then the same on every path, each store's wait lets kDepth - 1 stages stay
// in flight, and the fold runs between trips, outside the unrolled loop.
template <typename T, class Count, class Src, class Fold>
__device__ inline void tile_product(StageLds& lds, Acc& c, int G, Count count, Src src,
                                    Fold fold) {
  if (G <= 0) return;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  StageRegs ring[kDepth];
  // fetch cursor over the padded stage sequence
  int fg = 0, fl = 0, fn = count(0);
  const int last_g = G - 1, last_l = count(G - 1) - 1;
  auto fetch = [&](StageRegs& r) {
    const char *a, *b;
    int64_t lda, ldb;
    if (fg < G)
      src(fg, fl < fn ? fl : fn - 1, a, lda, b, ldb);
    else
      src(last_g, last_l, a, lda, b, ldb);
    stage_load(r, a, lda, b, ldb);
    if (fg < G && ++fl == (fn + kDepth - 1) / kDepth * kDepth) {
      fl = 0;
      if (++fg < G) fn = count(fg);
    }
  };
#pragma unroll
  for (int j = 0; j < kDepth; ++j) fetch(ring[j]);
  stage_store(lds, 0, ring[0]);
  fetch(ring[0]);
  stage_store(lds, 1, ring[1]);
  fetch(ring[1]);
  __syncthreads();
  Frag cur = frag_load(lds[0], wave, lane);
  int buf = 0;  // LDS buffer of the stage being multiplied
  for (int g = 0; g < G; ++g) {
    const int n = count(g), trips = (n + kDepth - 1) / kDepth;
    for (int trip = 0; trip < trips; ++trip) {
#pragma unroll
      for (int j = 0; j < kDepth; ++j) {
        const int l = trip * kDepth + j;
        const int buf1 = buf == kBuffers - 1 ? 0 : buf + 1;
        const int buf2 = buf1 == kBuffers - 1 ? 0 : buf1 + 1;
        const Frag nxt = frag_load(lds[buf1], wave, lane);
        if (l >= n) {  // a padding stage: A is zero
#pragma unroll
          for (int i = 0; i < 2; ++i) cur.x[i] = u32x4{0u, 0u, 0u, 0u};
        }
        Mma<T>::stage(c, cur);
        const int slot = (j + 2) % kDepth;  // static once the loop is unrolled
        stage_store(lds, buf2, ring[slot]);
        fetch(ring[slot]);
        __syncthreads();
        cur = nxt;
        buf = buf1;
      }
    }
    fold(g, c);
  }
}

// Everything a launch reads, by value.
struct RateArgs {
  wt_rate_tables tab;
  wt_rate_operand op;
  wt_rate_io io;
  int32_t t;
};

template <typename T>
__device__ inline T to_storage(float x) { return (T)x; }

// Rates of the state entering step 0 (and what the backward saves of it).
template <typename T>
__global__ __launch_bounds__(kThreads) void rate_init_kernel(RateArgs a) {
  const wt_rate_tables& tb = a.tab;
  const wt_rate_io& io = a.io;
  const int64_t N = tb.N, S = tb.S, T_ = io.T;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= io.B * N) return;
  const int64_t b = idx / N, n = idx - b * N;
  const float v = io.v[idx];
  const float r = tb.gain[n] * nonlin(tb.nonlinearity[n], v - tb.theta[n]);
  io.out[(b * T_) * N + n] = r;
  const int32_t pos = a.op.rpos ? a.op.rpos[n] : -1;
  if (pos >= 0) static_cast<T*>(a.op.rin)[b * a.op.K_rec_pad + pos] = to_storage<T>(r);
  if (io.v_saved) io.v_saved[(b * T_) * N + n] = v;
  if (io.I_saved)
    for (int64_t s = 0; s < S; ++s) io.I_saved[((b * T_) * N + n) * S + s] = io.I[(b * S + s) * N + n];
}

// Step t: a_k = r W_k for the recurrent pathways (segments of rin W), the input
// pathways' a_k from A_ff, then the currents, voltages and next rates. S (synapse
// types) is a template parameter: each lane keeps 16 x S targets.
template <typename T, int S>
__global__ __launch_bounds__(kThreads) void rate_step_kernel(RateArgs a) {
  __shared__ StageLds lds;
  const wt_rate_tables& tb = a.tab;
  const wt_rate_operand& op = a.op;
  const wt_rate_io& io = a.io;
  const int64_t N = tb.N, B = io.B, T_ = io.T, t = a.t;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wi = wave >> 1, wj = wave & 1;
  const int64_t n0 = (int64_t)blockIdx.x * kTile, b0 = (int64_t)blockIdx.y * kTile;
  const int64_t n = n0 + wj * 32 + (lane & 31);
  constexpr int kStageK = kStageBytes / (int)sizeof(T);
  const char* rin_b = reinterpret_cast<const char*>(
      static_cast<const T*>(op.rin) + ((t & 1) * op.B_pad + b0) * op.K_rec_pad);
  const char* Wt_n =
      reinterpret_cast<const char*>(static_cast<const T*>(op.Wt) + n0 * op.K_rec_pad);
  const int64_t ld = op.K_rec_pad * (int64_t)sizeof(T);

  float target[16][S];
#pragma unroll
  for (int v = 0; v < 16; ++v)
#pragma unroll
    for (int s = 0; s < S; ++s) target[v][s] = 0.0f;

  // k runs over the recurrent pathways' segments in order; at the end of each segment its
  // activation a_k enters the targets. Every segment's kernel scale for this tile's 64 targets, staged in LDS before the
  // product (the fold then issues no global load)
  __shared__ float s_jump[kMaxSeg][S][kTile];
  for (int i = threadIdx.x; i < op.n_seg * S * kTile; i += kThreads) {
    const int seg = i / (S * kTile), s = (i / kTile) % S, col = i % kTile;
    const int64_t tn = n0 + col;
    s_jump[seg][s][col] = tn < N ? tb.jump[((int64_t)op.seg[seg][2] * N + tn) * S + s] : 0.0f;
  }
  const int col = wj * 32 + (lane & 31);
  auto count = [&](int g) { return (int)((op.seg[g][1] - op.seg[g][0]) / kStageK); };
  auto src = [&](int g, int l, const char*& pa, int64_t& lda, const char*& pb, int64_t& ldb) {
    const int64_t off = (op.seg[g][0] / kStageK + l) * (int64_t)kStageBytes;
    pa = rin_b + off;
    pb = Wt_n + off;
    lda = ldb = ld;
  };
  __shared__ ReduceLds red;
  auto fold = [&](int g, Acc& c) {
    const int64_t path = op.seg[g][2];
    const f32x16 act = reduce(c, red, wave, lane);  // a_k of this wave's 32 x 32 block
    float jump[S];
#pragma unroll
    for (int q = 0; q < S; ++q) jump[q] = s_jump[g][q][col];
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int64_t b = b0 + wi * 32 + out_row(v, lane);
      if (io.A_saved && n < N && b < B) io.A_saved[((path * B + b) * T_ + t) * N + n] = act[v];
#pragma unroll
      for (int q = 0; q < S; ++q) target[v][q] = target[v][q] + act[v] * jump[q];
    }
  };
  // The state update of the lane's 16 trials. Its inputs do not depend on the product, so
  // every one of their loads is issued before it (their latency passes during the K
  // loop); after it, the arithmetic in registers, then every store.
  // With the voltages saved, the voltage entering this step is the saved one (written by
  // the previous step, or the first rates' launch), and the state v is written only
  // after the last step. A current whose decay is 0 is its target: its state is neither
  // read nor, before the last step, written.
  const bool in_range = n < N;
  const int64_t nn = in_range ? n : 0;
  auto row_b = [&](int v) { return b0 + wi * 32 + out_row(v, lane); };
  auto ok = [&](int v) { return in_range && row_b(v) < B; };
  auto el = [&](int v) { return (row_b(v) * T_ + t) * N + n; };  // (b, t, n) in (B, T, N)
  float decay[S], sign[S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    decay[s] = tb.decay[s];
    sign[s] = tb.sign[s];
  }
  const float beta = tb.beta[nn], theta = tb.theta[nn], gain = tb.gain[nn];
  const int code = tb.nonlinearity[nn];
  const int32_t pos = op.rpos ? op.rpos[nn] : -1;
  const bool has_ff = tb.K > tb.K_rec;
  float act0[16], jump0[S];  // the first input pathway
#pragma unroll
  for (int q = 0; q < S; ++q) jump0[q] = has_ff ? tb.jump[(tb.K_rec * N + nn) * S + q] : 0.0f;
  const float* __restrict__ A0 = io.A_ff;
  const float* __restrict__ v_saved_in = io.v_saved;
  const float* __restrict__ v_state_in = io.v;
  const float* __restrict__ I_in = io.I;
  float vv[16], I[16][S];
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const bool o = ok(v);
    const int64_t b = row_b(v);
    act0[v] = o && has_ff ? A0[el(v)] : 0.0f;
    vv[v] = !o ? 0.0f : v_saved_in ? v_saved_in[el(v)] : v_state_in[b * N + n];
#pragma unroll
    for (int s = 0; s < S; ++s)
      I[v][s] = o && decay[s] != 0.0f ? I_in[(b * S + s) * N + n] : 0.0f;
  }
  Acc c = {};
  tile_product<T>(lds, c, (int)op.n_seg, count, src, fold);
  if (n >= N) return;
  // the input pathways' activations, after the recurrent ones (pathway order)
  for (int64_t k = tb.K_rec; k < tb.K; ++k) {
    float act[16], jump[S];
    if (k == tb.K_rec) {
#pragma unroll
      for (int v = 0; v < 16; ++v) act[v] = act0[v];
#pragma unroll
      for (int q = 0; q < S; ++q) jump[q] = jump0[q];
    } else {
      const float* __restrict__ A = io.A_ff + (k - tb.K_rec) * B * T_ * N;
#pragma unroll
      for (int v = 0; v < 16; ++v) act[v] = ok(v) ? A[el(v)] : 0.0f;
#pragma unroll
      for (int q = 0; q < S; ++q) jump[q] = tb.jump[(k * N + n) * S + q];
    }
#pragma unroll
    for (int v = 0; v < 16; ++v)
#pragma unroll
      for (int q = 0; q < S; ++q) target[v][q] = target[v][q] + act[v] * jump[q];
    if (io.A_saved) {
      float* __restrict__ As = io.A_saved + k * B * T_ * N;
#pragma unroll
      for (int v = 0; v < 16; ++v)
        if (ok(v)) As[el(v)] = act[v];
    }
  }
  const bool last = t + 1 == T_;
  float r[16], x[16];
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    float I_syn = 0.0f;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const float d = decay[s];
      I[v][s] = d * I[v][s] + (1.0f - d) * target[v][s];
      I_syn = I_syn + I[v][s] * sign[s];
    }
    vv[v] = beta * vv[v] + (1.0f - beta) * I_syn;
    x[v] = vv[v] - theta;
  }
  nonlin_n<16>(code, gain, x, r);  // the lane's 16 trials share its neuron's nonlinearity
  float* __restrict__ out = io.out;
  float* __restrict__ v_saved_out = io.v_saved;
  float* __restrict__ v_state = io.v;
  float* __restrict__ I_state = io.I;
  T* __restrict__ rin_next = static_cast<T*>(op.rin) + ((t + 1) & 1) * op.B_pad * op.K_rec_pad;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    if (!ok(v)) continue;
    const int64_t b = b0 + wi * 32 + out_row(v, lane);
    if (!last) {
      out[el(v) + N] = r[v];
      if (pos >= 0) rin_next[b * op.K_rec_pad + pos] = to_storage<T>(r[v]);
      if (v_saved_out) v_saved_out[el(v) + N] = vv[v];
    }
    if (!v_saved_out || last) v_state[b * N + n] = vv[v];
#pragma unroll
    for (int s = 0; s < S; ++s)
      if (decay[s] != 0.0f || last) I_state[(b * S + s) * N + n] = I[v][s];
  }
  // what is saved or tracked (not on the plain forward path)
  if (io.target_saved || io.I_saved || io.track_v) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      if (!ok(v)) continue;
      const int64_t b = b0 + wi * 32 + out_row(v, lane);
#pragma unroll
      for (int s = 0; s < S; ++s) {
        if (io.target_saved) io.target_saved[el(v) * S + s] = target[v][s];
        if (io.I_saved && !last) io.I_saved[(el(v) + N) * S + s] = I[v][s];
      }
      if (io.track_v && (io.track_b < 0 || io.track_b == b)) {
        const int64_t row = ((io.track_b < 0 ? b : 0) * T_ + t) * N + n;
        io.track_v[row] = vv[v];
#pragma unroll
        for (int s = 0; s < S; ++s) io.track_I[row * S + s] = I[v][s];
      }
    }
  }
}

// Reverse, elementwise over (trial, neuron): (C) of step t+1 — the rate's gradient
// reaches the voltage entering step t+1 — then (A) of step t — the voltage's and
// currents' gradients reach this step's targets, hence dL/da_k of step t.
struct RateBackArgs {
  wt_rate_tables tab;
  wt_rate_operand op;
  wt_rate_back_io io;
  int32_t t;       // step of (A), or -1 for none
  int32_t t_rate;  // step of (C), or -1 for none
};

// V consecutive neurons of one trial per thread (V = 4: 16-byte loads and stores, when N
// is a multiple of 4 and every array is 16-byte aligned; V = 1 otherwise).
template <int V>
struct Vec {
  float x[V];
};
template <int V>
__device__ inline Vec<V> ldv(const float* p) {
  Vec<V> r;
  if constexpr (V == 4) {
    const float4 q = *reinterpret_cast<const float4*>(p);
    r.x[0] = q.x; r.x[1] = q.y; r.x[2] = q.z; r.x[3] = q.w;
  } else {
#pragma unroll
    for (int i = 0; i < V; ++i) r.x[i] = p[i];
  }
  return r;
}
template <int V>
__device__ inline void stv(float* p, const float (&x)[V]) {
  if constexpr (V == 4) {
    *reinterpret_cast<float4*>(p) = make_float4(x[0], x[1], x[2], x[3]);
  } else {
#pragma unroll
    for (int i = 0; i < V; ++i) p[i] = x[i];
  }
}

template <typename T, int S, int V>
__global__ __launch_bounds__(kThreads) void rate_back_elem_kernel(RateBackArgs a) {
  const wt_rate_tables& tb = a.tab;
  const wt_rate_back_io& io = a.io;
  const int64_t N = tb.N, K = tb.K, B = io.B, T_ = io.T;
  const int64_t idx = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * V;  // (b, n) flat
  if (idx >= B * N) return;
  const int64_t b = idx / N, n = idx - b * N;  // n .. n + V - 1, one trial
  const bool rate = a.t_rate >= 0, adj = a.t >= 0;
  const int64_t u = a.t_rate, t = a.t;
  const int64_t el_u = (b * T_ + u) * N + n, el_t = (b * T_ + t) * N + n;
  // Every load first — none of them depends on another, and the arrays do not alias —
  // then the arithmetic, then the stores: one round trip to memory per thread.
  float* __restrict__ lam_v = io.lam_v;
  float* __restrict__ lam_I = io.lam_I;
  const float* __restrict__ grad_out = io.grad_out;
  const float* __restrict__ d_rate = io.d_rate;
  const float* __restrict__ v_saved = io.v_saved;
  Vec<V> lv = ldv<V>(lam_v + idx), dr = {}, vs = {};
  if (rate) {
    dr = ldv<V>(grad_out + el_u);
    if (d_rate) {
      const Vec<V> d = ldv<V>(d_rate + b * N + n);
#pragma unroll
      for (int i = 0; i < V; ++i) dr.x[i] = dr.x[i] + d.x[i];
    }
    vs = ldv<V>(v_saved + el_u);
  }
  const Vec<V> theta = ldv<V>(tb.theta + n), gain = ldv<V>(tb.gain + n),
               beta = ldv<V>(tb.beta + n);
  int code[V];
#pragma unroll
  for (int i = 0; i < V; ++i) code[i] = tb.nonlinearity[n + i];
  float decay[S], sign[S], lamI[S][V];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    decay[s] = tb.decay[s];
    sign[s] = tb.sign[s];
  }
#pragma unroll
  for (int s = 0; s < S; ++s) {  // a current whose decay is 0 passes no adjoint back in time
    const Vec<V> l = adj && decay[s] != 0.0f ? ldv<V>(lam_I + (b * S + s) * N + n) : Vec<V>{};
#pragma unroll
    for (int i = 0; i < V; ++i) lamI[s][i] = l.x[i];
  }
  constexpr int kChunk = 2;
  float jump[kChunk][V][S];  // jump[k][n + i][s], S * V consecutive floats per pathway
  auto load_jump = [&](int64_t k0) {
#pragma unroll
    for (int c = 0; c < kChunk; ++c)
#pragma unroll
      for (int i = 0; i < V; ++i)
#pragma unroll
        for (int s = 0; s < S; ++s)
          jump[c][i][s] = adj && k0 + c < K ? tb.jump[((k0 + c) * N + n + i) * S + s] : 0.0f;
  };
  load_jump(0);

  float lvx[V];
#pragma unroll
  for (int i = 0; i < V; ++i) lvx[i] = lv.x[i];
  if (rate) {  // (C): v_u enters r_u; lv holds beta dL/dv_{u+1} already
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const float x = vs.x[i] - theta.x[i];
      const float gf = dr.x[i] * gain.x[i];
      const float fp = nonlin_grad(code[i], x);
      lvx[i] = lvx[i] + gf * fp;
      if (io.acc_theta) io.acc_theta[idx + i] -= gf * fp;
      if (io.acc_gain) io.acc_gain[idx + i] += dr.x[i] * nonlin(code[i], x);
    }
  }
  if (adj) {  // (A) of step t: v_{t+1} = beta v_t + (1 - beta) sum_s sign_s I_{t+1,s}
    float dtarget[S][V];
#pragma unroll
    for (int i = 0; i < V; ++i) {
      float I_next_syn = 0.0f;
#pragma unroll
      for (int s = 0; s < S; ++s) {
        if (io.acc_beta) {
          const float I_next = t + 1 < T_ ? io.I_saved[(el_t + i + N) * S + s]
                                          : io.I_final[(b * S + s) * N + n + i];
          I_next_syn = I_next_syn + I_next * sign[s];
        }
        const float dI = lamI[s][i] + lvx[i] * (1.0f - beta.x[i]) * sign[s];
        dtarget[s][i] = dI * (1.0f - decay[s]);
        lamI[s][i] = dI * decay[s];
        if (io.acc_decay)
          io.acc_decay[(b * S + s) * N + n + i] +=
              dI * (io.I_saved[(el_t + i) * S + s] - io.target_saved[(el_t + i) * S + s]);
      }
      if (io.acc_beta) io.acc_beta[idx + i] += lvx[i] * (v_saved[el_t + i] - I_next_syn);
    }
    // dL/da_k = sum_s dtarget_s jump_k[s], kChunk pathways at a time
    float* __restrict__ grad_A = io.grad_A;
    T* __restrict__ gA_op = static_cast<T*>(io.gA_op);
    for (int64_t k0 = 0; k0 < K; k0 += kChunk) {
      if (k0 > 0) load_jump(k0);
#pragma unroll
      for (int c = 0; c < kChunk; ++c) {
        const int64_t k = k0 + c;
        if (k >= K) break;
        float g[V];
#pragma unroll
        for (int i = 0; i < V; ++i) {
          g[i] = 0.0f;
#pragma unroll
          for (int s = 0; s < S; ++s) g[i] = g[i] + dtarget[s][i] * jump[c][i][s];
        }
        stv<V>(grad_A + ((k * B + b) * T_ + t) * N + n, g);
        if (k < tb.K_rec) {
          T* dst = gA_op + (k * a.op.B_pad + b) * a.op.N_pad + n;
#pragma unroll
          for (int i = 0; i < V; ++i) dst[i] = to_storage<T>(g[i]);
        }
        if (io.acc_scale) {
          float m[V];
#pragma unroll
          for (int i = 0; i < V; ++i) {
            m[i] = 0.0f;
#pragma unroll
            for (int s = 0; s < S; ++s) m[i] = m[i] + dtarget[s][i] * tb.made[k * S + s];
            io.acc_scale[(k * B + b) * N + n + i] +=
                m[i] * io.A_saved[((k * B + b) * T_ + t) * N + n + i];
          }
        }
      }
    }
#pragma unroll
    for (int s = 0; s < S; ++s)
      if (decay[s] != 0.0f) {
        float l[V];
#pragma unroll
        for (int i = 0; i < V; ++i) l[i] = lamI[s][i];
        stv<V>(lam_I + (b * S + s) * N + n, l);
      }
#pragma unroll
    for (int i = 0; i < V; ++i) lvx[i] = lvx[i] * beta.x[i];  // dL/dv_t before its rate's term
  }
  stv<V>(lam_v + idx, lvx);
}

// Reverse product of step t: d_rate[b, neuron of row j] = sum_n dL/da_k[b, n] W[j, n] for
// the recurrent rows j of pathway k (the rates' gradient through the recurrence). W's
// rows are k-contiguous along n: the tile product's second operand as it is.
template <typename T>
__global__ __launch_bounds__(kThreads) void rate_back_gemm_kernel(RateBackArgs a) {
  __shared__ StageLds lds;
  const wt_rate_operand& op = a.op;
  const wt_rate_back_io& io = a.io;
  const int64_t N = a.tab.N, B = io.B;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t j0 = (int64_t)blockIdx.x * kTile, b0 = (int64_t)blockIdx.y * kTile;
  // the recurrent segment holding rows [j0, j0 + 64): segments are whole tiles
  int64_t path = -1;
  for (int g = 0; g < op.n_seg; ++g)
    if (!op.seg[g][3] && j0 >= op.seg[g][0] && j0 < op.seg[g][1]) path = op.seg[g][2];
  if (path < 0) return;
  constexpr int kStageK = kStageBytes / (int)sizeof(T);
  const char* gA = reinterpret_cast<const char*>(static_cast<const T*>(io.gA_op) +
                                                 (path * op.B_pad + b0) * op.N_pad);
  const char* Wj = reinterpret_cast<const char*>(static_cast<const T*>(op.W) + j0 * op.N_pad);
  const int64_t ld = op.N_pad * (int64_t)sizeof(T);
  __shared__ ReduceLds red;
  Acc acc = {};
  tile_product<T>(
      lds, acc, 1, [&](int) { return (int)(op.N_pad / kStageK); },
      [&](int, int l, const char*& pa, int64_t& lda, const char*& pb, int64_t& ldb) {
        pa = gA + (int64_t)l * kStageBytes;
        pb = Wj + (int64_t)l * kStageBytes;
        lda = ldb = ld;
      },
      [](int, Acc&) {});
  const f32x16 c = reduce(acc, red, wave, lane);
  const int wi = wave >> 1, wj = wave & 1;
  const int64_t j = j0 + wj * 32 + (lane & 31);
  const int32_t neuron = op.src_of[j];
  if (neuron < 0) return;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int64_t b = b0 + wi * 32 + out_row(v, lane);
    if (b < B) io.d_rate[b * N + neuron] = c[v];
  }
}

// ---------------------------------------------------------------------------------
// The forward's split product, for a drive of one recurrent pathway: P[z] = A[:, slice z]
// Bt[:, slice z]^T in float32, 128 x 128 outputs per workgroup and the k dimension cut
// into KS slices of whole stages (grid: output columns / 128, rows / 128, KS). Against the
// 64 x 64 tiles of the fused step, every staged byte feeds twice the matrix-core work
// (each CU fetches 512 KB per step at configuration 4's shape instead of 1 MB), and the
// KS slices keep every CU busy (256 x 4096 outputs: 64 tiles x 4 slices). The update
// launch that follows sums the KS partials of an output in slice order.
//
// A stage is 128 bytes of k of 128 rows per operand (16 KB each): thread t fetches chunk
// t % 8 of rows t / 8 + 32m, m < 4. Stages are fetched kSplitDepth ahead into a ring of
// registers and stored to LDS in the swizzled layout of the fused tiles (row r's chunk c
// in slot c ^ swz(r); rows r and r + 32m share swz). Wave w owns the 64 x 64 block (w / 2,
// w % 2) of the tile — 2 x 2 MFMA blocks of 32 x 32 — over the whole stage, so no partials
// cross waves. Three LDS buffers: stage s + 2 is stored while stage s is multiplied; one
// barrier per stage.
// ---------------------------------------------------------------------------------

constexpr int kBig = 128;
constexpr int kSplitDepth = 4;
typedef u32x4 BigLds[kBuffers][2][kBig * 8];

struct BigRegs {
  u32x4 a[4], b[4];
};

struct SplitArgs {
  const char* A;  // row m0 of the tile, column 0 of the slice (bytes)
  const char* B;
  int64_t lda, ldb;  // row pitches in bytes
  float* P;          // [KS][M_pad][ldp]
  int64_t ldp, M_pad;
  int32_t stages;    // per slice
};

template <typename T>
__global__ __launch_bounds__(kThreads) void split_product_kernel(SplitArgs sa) {
  __shared__ BigLds lds;
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63, wi = wave >> 1, wj = wave & 1;
  const int64_t m0 = (int64_t)blockIdx.y * kBig, n0 = (int64_t)blockIdx.x * kBig;
  const int n_st = sa.stages;
  const int64_t k0 = (int64_t)blockIdx.z * n_st * kStageBytes;
  const char* A = sa.A + m0 * sa.lda + k0;
  const char* Bt = sa.B + n0 * sa.ldb + k0;
  const int row = t >> 3, off = (t & 7) * 16, slot_w = (t & 7) ^ swz(row);
  // a stage's operands (past the last stage: the last one again, never multiplied)
  auto fetch = [&](BigRegs& r, int st) {
    const int64_t c = (int64_t)(st < n_st ? st : n_st - 1) * kStageBytes + off;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      r.a[m] = gload16(A + (row + 32 * m) * sa.lda + c);
      r.b[m] = gload16(Bt + (row + 32 * m) * sa.ldb + c);
    }
  };
  auto store = [&](int buf, const BigRegs& r) {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      lds[buf][0][(row + 32 * m) * 8 + slot_w] = r.a[m];
      lds[buf][1][(row + 32 * m) * 8 + slot_w] = r.b[m];
    }
  };
  // the wave's fragments: rows wi * 64 + 32 i + lane % 32 of A, wj * 64 + 32 j + lane % 32
  // of Bt; k-step kk takes chunk 2 kk + lane / 32
  const int r = lane & 31, h = lane >> 5, sw = swz(r);
  // a stage's fragments, all four k-steps
  auto read = [&](int buf, Frag (&f)[4]) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int slot = (2 * kk + h) ^ sw;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        f[kk].x[i] = lds[buf][0][(wi * 64 + 32 * i + r) * 8 + slot];
        f[kk].y[i] = lds[buf][1][(wj * 64 + 32 * i + r) * 8 + slot];
      }
    }
  };
  Acc c = {};
  BigRegs ring[kSplitDepth];
#pragma unroll
  for (int j = 0; j < kSplitDepth; ++j) fetch(ring[j], j);
  store(0, ring[0]);
  fetch(ring[0], kSplitDepth);
  store(1, ring[1]);
  fetch(ring[1], kSplitDepth + 1);
  __syncthreads();
  Frag cur[4];
  read(0, cur);
  // Whole trips of kSplitDepth stages; past the last stage the multiply takes zeros, so
  // every path issues the same loads and each store's wait leaves the later stages'
  // loads in flight. Stage s + 1's fragments (its buffer complete since the barrier
  // before) are read while stage s's MFMAs run: with one wave per SIMD nothing else
  // hides the LDS latency.
  const int trips = (n_st + kSplitDepth - 1) / kSplitDepth;
  for (int trip = 0; trip < trips; ++trip) {
#pragma unroll
    for (int j = 0; j < kSplitDepth; ++j) {
      const int st = trip * kSplitDepth + j;
      Frag nxt[4];
      read((st + 1) % kBuffers, nxt);
      if (st >= n_st) {  // a padding stage: A is zero (no branch around the MFMAs, which
                         // would let the reads above sink below them)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
          for (int i = 0; i < 2; ++i) cur[kk].x[i] = u32x4{0u, 0u, 0u, 0u};
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) Mma<T>::stage(c, cur[kk]);
      const int slot = (j + 2) % kSplitDepth;  // static once unrolled
      store((st + 2) % kBuffers, ring[slot]);
      fetch(ring[slot], st + 2 + kSplitDepth);
      __syncthreads();
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) cur[kk] = nxt[kk];
    }
  }
  float* P = sa.P + ((int64_t)blockIdx.z * sa.M_pad + m0) * sa.ldp + n0;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v)
        P[(int64_t)(wi * 64 + 32 * i + out_row(v, lane)) * sa.ldp + wj * 64 + 32 * j + (lane & 31)] =
            c[i][j][v];
}

// The k slices of a split product of `tiles` output tiles over `stages` stages: doubled
// while a slice keeps whole stages and the workgroups stay within one per CU (256), at
// most 4.
static int split_slices(int64_t tiles, int64_t stages) {
  int ks = 1;
  while (ks < kMaxSlices && tiles * ks * 2 <= 256 && stages % (ks * 2) == 0) ks *= 2;
  return ks;
}

// Whether a call takes the split products: one recurrent pathway, every padded size a
// multiple of the 128-wide tiles.
static bool split_applies(const wt_rate_operand& op) {
  return op.n_seg == 1 && op.K_rec_pad > 0 && op.B_pad % kBig == 0 && op.N_pad % kBig == 0 &&
         op.K_rec_pad % kBig == 0;
}

template <typename T>
static int forward_slices(const wt_rate_operand& op) {
  constexpr int kStageK = kStageBytes / (int)sizeof(T);
  return split_slices((op.N_pad / kBig) * (op.B_pad / kBig), op.K_rec_pad / kStageK);
}

// Step t after a split product: per (trial, neuron), the recurrent activation (the KS
// partials summed in slice order), the input pathways', then the currents, voltage and
// next rate — the fused step's epilogue, one element per thread (neurons fastest).
// Every load is issued before the first store: on gfx950 one counter tracks a wave's
// outstanding loads and stores alike, so a load placed after a store (the compiler keeps
// the program order where it cannot rule out aliasing) makes its use wait for the store.
constexpr int kUpdateFF = 2;  // input pathways held in registers (the rest read in turn)

template <typename T, int S>
__global__ __launch_bounds__(kThreads) void rate_update_kernel(RateArgs a, const float* P,
                                                               int KS) {
  const wt_rate_tables& tb = a.tab;
  const wt_rate_operand& op = a.op;
  const wt_rate_io& io = a.io;
  const int64_t N = tb.N, B = io.B, T_ = io.T, t = a.t;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= B * N) return;
  const int64_t b = idx / N, n = idx - b * N;
  const int64_t el = (b * T_ + t) * N + n;
  const int64_t path = op.seg[0][2];
  const int64_t K_ff = tb.K - tb.K_rec;
  // ---- loads ----
  const float* q = P + b * op.N_pad + n;
  const int64_t slice = op.B_pad * op.N_pad;
  float p[kMaxSlices];
#pragma unroll
  for (int ks = 0; ks < kMaxSlices; ++ks) p[ks] = ks < KS ? q[ks * slice] : 0.0f;
  float jr[S], dec[S], sgn[S], I_prev[S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    jr[s] = tb.jump[(path * N + n) * S + s];
    dec[s] = tb.decay[s];
    sgn[s] = tb.sign[s];
  }
  float ak[kUpdateFF], jf[kUpdateFF][S];
#pragma unroll
  for (int j = 0; j < kUpdateFF; ++j) {
    const int64_t k = tb.K_rec + j;
    ak[j] = j < K_ff ? io.A_ff[j * B * T_ * N + el] : 0.0f;
#pragma unroll
    for (int s = 0; s < S; ++s) jf[j][s] = j < K_ff ? tb.jump[(k * N + n) * S + s] : 0.0f;
  }
  float v = io.v_saved ? io.v_saved[el] : io.v[b * N + n];
#pragma unroll
  for (int s = 0; s < S; ++s) I_prev[s] = dec[s] != 0.0f ? io.I[(b * S + s) * N + n] : 0.0f;
  const float beta = tb.beta[n], gain = tb.gain[n], theta = tb.theta[n];
  const int32_t code = tb.nonlinearity[n];
  const int32_t pos = op.rpos ? op.rpos[n] : -1;
  // ---- arithmetic, in the reference's order ----
  float act = p[0];
#pragma unroll
  for (int ks = 1; ks < kMaxSlices; ++ks)
    if (ks < KS) act = act + p[ks];
  float target[S];
#pragma unroll
  for (int s = 0; s < S; ++s) target[s] = 0.0f + act * jr[s];
#pragma unroll
  for (int j = 0; j < kUpdateFF; ++j) {  // the input pathways, in order
    if (j >= K_ff) break;
#pragma unroll
    for (int s = 0; s < S; ++s) target[s] = target[s] + ak[j] * jf[j][s];
  }
  // ---- stores (and the input pathways past the registers: loads after stores) ----
  if (io.A_saved) {
    io.A_saved[((path * B + b) * T_ + t) * N + n] = act;
#pragma unroll
    for (int j = 0; j < kUpdateFF; ++j)
      if (j < K_ff) io.A_saved[(tb.K_rec + j) * B * T_ * N + el] = ak[j];
  }
  for (int64_t k = tb.K_rec + kUpdateFF; k < tb.K; ++k) {
    const float a_k = io.A_ff[(k - tb.K_rec) * B * T_ * N + el];
#pragma unroll
    for (int s = 0; s < S; ++s) target[s] = target[s] + a_k * tb.jump[(k * N + n) * S + s];
    if (io.A_saved) io.A_saved[k * B * T_ * N + el] = a_k;
  }
  const bool last = t + 1 == T_;
  float I[S], I_syn = 0.0f;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    I[s] = dec[s] * I_prev[s] + (1.0f - dec[s]) * target[s];
    I_syn = I_syn + I[s] * sgn[s];
  }
  v = beta * v + (1.0f - beta) * I_syn;
  const float r = gain * nonlin(code, v - theta);
  if (!last) {
    io.out[el + N] = r;
    if (pos >= 0)
      static_cast<T*>(op.rin)[(((t + 1) & 1) * op.B_pad + b) * op.K_rec_pad + pos] =
          to_storage<T>(r);
    if (io.v_saved) io.v_saved[el + N] = v;
  }
  if (!io.v_saved || last) io.v[b * N + n] = v;
#pragma unroll
  for (int s = 0; s < S; ++s)
    if (dec[s] != 0.0f || last) io.I[(b * S + s) * N + n] = I[s];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    if (io.target_saved) io.target_saved[el * S + s] = target[s];
    if (io.I_saved && !last) io.I_saved[(el + N) * S + s] = I[s];
  }
  if (io.track_v && (io.track_b < 0 || io.track_b == b)) {
    const int64_t row = ((io.track_b < 0 ? b : 0) * T_ + t) * N + n;
    io.track_v[row] = v;
#pragma unroll
    for (int s = 0; s < S; ++s) io.track_I[row * S + s] = I[s];
  }
}

template <typename T>
static hipError_t forward_impl(const RateArgs& base, hipStream_t stream) {
  RateArgs a = base;
  const int64_t BN = a.io.B * a.tab.N;
  a.t = 0;
  hipLaunchKernelGGL(rate_init_kernel<T>, dim3((unsigned)((BN + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, stream, a);
  const dim3 grid((unsigned)(a.op.N_pad / kTile), (unsigned)(a.op.B_pad / kTile));
  void (*step)(RateArgs) = nullptr;
  switch (a.tab.S) {
    case 1: step = rate_step_kernel<T, 1>; break;
    case 2: step = rate_step_kernel<T, 2>; break;
    case 3: step = rate_step_kernel<T, 3>; break;
    case 4: step = rate_step_kernel<T, 4>; break;
    case 5: step = rate_step_kernel<T, 5>; break;
    case 6: step = rate_step_kernel<T, 6>; break;
    case 7: step = rate_step_kernel<T, 7>; break;
    case 8: step = rate_step_kernel<T, 8>; break;
    default: return hipErrorInvalidValue;
  }
  if (a.io.split && split_applies(a.op)) {
    void (*update)(RateArgs, const float*, int) = nullptr;
    switch (a.tab.S) {
      case 1: update = rate_update_kernel<T, 1>; break;
      case 2: update = rate_update_kernel<T, 2>; break;
      case 3: update = rate_update_kernel<T, 3>; break;
      case 4: update = rate_update_kernel<T, 4>; break;
      case 5: update = rate_update_kernel<T, 5>; break;
      case 6: update = rate_update_kernel<T, 6>; break;
      case 7: update = rate_update_kernel<T, 7>; break;
      case 8: update = rate_update_kernel<T, 8>; break;
      default: return hipErrorInvalidValue;
    }
    constexpr int kStageK = kStageBytes / (int)sizeof(T);
    const int KS = forward_slices<T>(a.op);
    const dim3 sgrid((unsigned)(a.op.N_pad / kBig), (unsigned)(a.op.B_pad / kBig), (unsigned)KS);
    const dim3 ugrid((unsigned)((BN + kThreads - 1) / kThreads));
    SplitArgs sa = {};
    sa.B = static_cast<const char*>(a.op.Wt);
    sa.lda = sa.ldb = a.op.K_rec_pad * (int64_t)sizeof(T);
    sa.P = a.io.split;
    sa.ldp = a.op.N_pad;
    sa.M_pad = a.op.B_pad;
    sa.stages = (int32_t)(a.op.K_rec_pad / kStageK / KS);
    for (int64_t t = 0; t < a.io.T; ++t) {
      a.t = (int32_t)t;
      sa.A = reinterpret_cast<const char*>(static_cast<const T*>(a.op.rin) +
                                           (t & 1) * a.op.B_pad * a.op.K_rec_pad);
      hipLaunchKernelGGL(split_product_kernel<T>, sgrid, dim3(kThreads), 0, stream, sa);
      hipLaunchKernelGGL(update, ugrid, dim3(kThreads), 0, stream, a,
                         static_cast<const float*>(a.io.split), KS);
    }
    return hipGetLastError();
  }
  for (int64_t t = 0; t < a.io.T; ++t) {
    a.t = (int32_t)t;
    hipLaunchKernelGGL(step, grid, dim3(kThreads), 0, stream, a);
  }
  return hipGetLastError();
}

template <typename T>
static hipError_t backward_impl(const RateBackArgs& base, hipStream_t stream) {
  RateBackArgs a = base;
  const int64_t BN = a.io.B * a.tab.N;
  const dim3 egrid_1((unsigned)((BN + kThreads - 1) / kThreads));
  const dim3 egrid_4((unsigned)((BN / 4 + kThreads - 1) / kThreads));
  const dim3 ggrid((unsigned)(a.op.K_rec_pad / kTile), (unsigned)(a.op.B_pad / kTile));
  const bool rec = a.tab.K_rec > 0 && a.op.K_rec_pad > 0;
  void (*elem)(RateBackArgs) = nullptr;
  // four neurons per thread when every (., N) row and array is 16-byte aligned
  auto al = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  const wt_rate_back_io& q = a.io;
  const bool v4 = a.tab.N % 4 == 0 && al(q.grad_out) && al(q.v_saved) && al(q.lam_v) &&
                  al(q.lam_I) && al(q.grad_A) && (!q.d_rate || al(q.d_rate)) &&
                  al(a.tab.theta) && al(a.tab.gain) && al(a.tab.beta);
  const int vw = v4 ? 4 : 1;
  switch (a.tab.S * 8 + vw) {
#define WT_ELEM(SS)                                                     \
    case SS * 8 + 1: elem = rate_back_elem_kernel<T, SS, 1>; break; \
    case SS * 8 + 4: elem = rate_back_elem_kernel<T, SS, 4>; break;
    WT_ELEM(1) WT_ELEM(2) WT_ELEM(3) WT_ELEM(4) WT_ELEM(5) WT_ELEM(6) WT_ELEM(7) WT_ELEM(8)
#undef WT_ELEM
    default: return hipErrorInvalidValue;
  }
  for (int64_t t = a.io.T - 1; t >= -1; --t) {
    a.t = (int32_t)t;
    a.t_rate = t + 1 < a.io.T ? (int32_t)(t + 1) : -1;
    hipLaunchKernelGGL(elem, vw == 4 ? egrid_4 : egrid_1, dim3(kThreads), 0, stream, a);
    if (t >= 0 && rec)
      hipLaunchKernelGGL(rate_back_gemm_kernel<T>, ggrid, dim3(kThreads), 0, stream, a);
  }
  return hipGetLastError();
}

static bool operand_ok(const wt_rate_tables* tb, const wt_rate_operand* op, int64_t B) {
  if (op->dtype != 0 && op->dtype != 1) return false;
  if (op->B_pad < B || op->B_pad % kTile || op->N_pad < tb->N || op->N_pad % kTile) return false;
  if (op->K_rec_pad % kTile || op->n_seg < 0 || op->n_seg > kMaxSeg) return false;
  int64_t end = 0;  // segments tile [0, K_rec_pad) in order, one per recurrent pathway
  for (int64_t g = 0; g < op->n_seg; ++g) {
    const int32_t* s = op->seg[g];
    if (s[0] != end || s[1] <= s[0] || s[1] % kTile || s[3] != 0) return false;
    if (s[2] < 0 || s[2] >= tb->K_rec) return false;
    end = s[1];
  }
  if (end != op->K_rec_pad) return false;
  return op->K_rec_pad == 0 || (op->W && op->Wt && op->rin && op->rpos);
}

}  // namespace rate
}  // namespace wt

using namespace wt::rate;

extern "C" int wt_rate_forward(const wt_rate_tables* tab, const wt_rate_operand* op,
                               const wt_rate_io* io, wt_stream_t stream) {
  if (!tab || !op || !io || !io->v || !io->I || !io->out) return hipErrorInvalidValue;
  if (tab->S < 1 || tab->S > kMaxS || tab->K < 0 || tab->K_rec < 0 || tab->K_rec > tab->K)
    return hipErrorInvalidValue;
  if (!operand_ok(tab, op, io->B)) return hipErrorInvalidValue;
  if (tab->K > tab->K_rec && !io->A_ff) return hipErrorInvalidValue;
  if ((io->track_v != nullptr) != (io->track_I != nullptr)) return hipErrorInvalidValue;
  if (io->B * tab->N == 0 || io->T == 0) return hipSuccess;
  RateArgs a = {};
  a.tab = *tab;
  a.op = *op;
  a.io = *io;
  return op->dtype == 1 ? forward_impl<__bf16>(a, (hipStream_t)stream)
                        : forward_impl<float>(a, (hipStream_t)stream);
}

extern "C" int wt_rate_backward(const wt_rate_tables* tab, const wt_rate_operand* op,
                                const wt_rate_back_io* io, wt_stream_t stream) {
  if (!tab || !op || !io || !io->grad_out || !io->v_saved || !io->lam_v || !io->lam_I ||
      !io->grad_A || !io->I_final)
    return hipErrorInvalidValue;
  if (tab->S < 1 || tab->S > kMaxS || tab->K < 0 || tab->K_rec < 0 || tab->K_rec > tab->K)
    return hipErrorInvalidValue;
  if (!operand_ok(tab, op, io->B)) return hipErrorInvalidValue;
  if (tab->K_rec > 0 && (!io->gA_op || !io->d_rate || !op->src_of)) return hipErrorInvalidValue;
  if ((io->acc_decay || io->acc_scale) && (!io->I_saved || !io->target_saved))
    return hipErrorInvalidValue;
  if (io->acc_scale && !io->A_saved) return hipErrorInvalidValue;
  if (io->acc_beta && io->T > 1 && !io->I_saved) return hipErrorInvalidValue;
  if (io->B * tab->N == 0 || io->T == 0) return hipSuccess;
  RateBackArgs a = {};
  a.tab = *tab;
  a.op = *op;
  a.io = *io;
  return op->dtype == 1 ? backward_impl<__bf16>(a, (hipStream_t)stream)
                        : backward_impl<float>(a, (hipStream_t)stream);
}

extern "C" int64_t wt_rate_split_bytes(const wt_rate_tables* tab, const wt_rate_operand* op,
                                       int64_t B) {
  if (!tab || !op || !operand_ok(tab, op, B) || tab->K_rec < 1 || !split_applies(*op)) return 0;
  const int64_t ks = op->dtype == 1 ? forward_slices<__bf16>(*op) : forward_slices<float>(*op);
  return ks * op->B_pad * op->N_pad * 4;
}

// ---- hi = bf16(x), lo = bf16(x - hi): x = hi + lo to 2^-17 relative (x - hi is exact in
// float32). Eight values per thread (two 16-byte loads, two 16-byte stores); the tail
// one at a time.
namespace wt {
namespace rate {
__global__ void split_bf16_kernel(const float* __restrict__ x, int64_t n, __bf16* __restrict__ hi,
                                  __bf16* __restrict__ lo) {
  const int64_t i0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (i0 + 8 <= n) {
    const float4 a = *reinterpret_cast<const float4*>(x + i0);
    const float4 b = *reinterpret_cast<const float4*>(x + i0 + 4);
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    __bf16 h[8], l[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      h[u] = (__bf16)v[u];
      l[u] = (__bf16)(v[u] - (float)h[u]);
    }
    *reinterpret_cast<uint4*>(hi + i0) = *reinterpret_cast<const uint4*>(h);
    *reinterpret_cast<uint4*>(lo + i0) = *reinterpret_cast<const uint4*>(l);
  } else {
    for (int64_t i = i0; i < n; ++i) {
      const __bf16 h = (__bf16)x[i];
      hi[i] = h;
      lo[i] = (__bf16)(x[i] - (float)h);
    }
  }
}
}  // namespace rate
}  // namespace wt

extern "C" int wt_split_bf16(const float* x, int64_t n, void* hi, void* lo, wt_stream_t stream) {
  if (n < 0) return hipErrorInvalidValue;
  if (n == 0) return hipSuccess;
  if (!x || !hi || !lo) return hipErrorInvalidValue;
  // 16-byte vectors: every array 16-byte aligned
  if (((uintptr_t)x | (uintptr_t)hi | (uintptr_t)lo) & 15) return hipErrorInvalidValue;
  const int64_t threads = (n + 7) / 8;
  const int block = 256;
  hipLaunchKernelGGL(wt::rate::split_bf16_kernel, dim3((unsigned)((threads + block - 1) / block)),
                     dim3(block), 0, (hipStream_t)stream, x, n, static_cast<__bf16*>(hi),
                     static_cast<__bf16*>(lo));
  return hipGetLastError();
}
