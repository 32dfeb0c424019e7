// Convolution kernels for gfx950 (CDNA4): implicit-GEMM conv on MFMA, first conv (Cin = 3)
// and depthwise conv.
//
// GEMM view of a conv (the reference's k_conv_mma contract, engine/engine.cu:250-483):
//   D[n][m] = sum_k W[n][k] * A[m][k]
//   m = pixel (img, oy, ox) in [0, B*Ho*Wo), n = output channel, k = (ky, kx, ci) flat
//   ("dense K": no per-tap padding), W = OHWI weights, A = the im2col row of pixel m,
//   gathered on the fly from the NHWC input (no im2col buffer).
// Epilogue: + bias, SiLU (act 1), + residual (act first, then +res), fp16 store into a
// strided channel slice, so concat is zero-copy.  Accumulation is always fp32.
//
// MI355X design:
//  * v_mfma_f32_16x16x32_f16: the weight tile is the MFMA A operand (16 channels x 32 k)
//    and the pixel tile the B operand (32 k x 16 pixels), so each lane ends up holding
//    four consecutive output channels of one pixel -> 8-byte NHWC stores, contiguous
//    per pixel across the four lane groups.
//  * K is staged BK halves (32, 64 or 128: one to four MFMA steps) at a time through
//    double-buffered LDS.  The next stage's 16-byte global loads are issued into
//    registers before the MFMAs of the current stage, so one barrier per stage hides the
//    global latency behind matrix work; small convs (batch 1) use deep stages so each
//    barrier carries many loads in flight, large convs use wide tiles.
//  * LDS rows hold BK halves as 16-byte chunks; chunk c of row r is stored at
//    c ^ f(r) so the 16-byte MFMA operand reads of 8 consecutive rows (one LDS clock of
//    a ds_read_b128) hit distinct 16-byte bank groups.
//  * Block order: the linear block id is remapped so that the N tiles of one M tile are
//    consecutive in dispatch order (the activation tile, the larger operand, is then
//    re-read from L2 instead of HBM), and consecutive ids are first grouped per XCD
//    (dispatch is round-robin over the 8 XCDs, each with its own L2).
//  * Tile shapes are template parameters; the host picks one per conv by heuristic and
//    a startup autotuner.
#include "engine.hpp"

namespace yolo {

typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int NUM_XCD = 8;

template <int CPR>
__device__ __forceinline__ int swz(int row, int c) {
  // CPR = 16-byte chunks per row; 8 consecutive rows must land on distinct chunk slots
  // of a 128-byte window
  if constexpr (CPR >= 8) return row * CPR + (c ^ (row & 7));
  else return row * CPR + (c ^ ((row >> 1) & (CPR - 1)));
}

__device__ __forceinline__ float silu(float v) { return v / (1.0f + __expf(-v)); }

template <int BM, int BN, int WM, int WN, int BK, bool KONE>
__global__ __launch_bounds__(64 * WM * WN) void k_conv_gemm(
    View x, View y, View r, const f16* __restrict__ w, const float* __restrict__ bias,
    int ksz, int cs, int cp, int act, int M, int N, int Ktot, int mtiles, int ntiles) {
  constexpr int NT = 64 * WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN;  // wave tile: pixels x channels
  constexpr int FM = TM / 16, FN = TN / 16;
  constexpr int CPR = BK / 8;                // 16-byte chunks per LDS row
  constexpr int KS = BK / 32;                // MFMA steps per stage
  static_assert(TM % 16 == 0 && TN % 16 == 0, "wave tile must be a multiple of 16");
  static_assert(NT % CPR == 0, "chunk column must be fixed per thread");
  constexpr int AL = (BM * CPR + NT - 1) / NT;  // 16-byte A chunks per thread per stage
  constexpr int BL = (BN * CPR + NT - 1) / NT;

  __shared__ f16x8 sA[2][BM * CPR];
  __shared__ f16x8 sB[2][BN * CPR];

  // ---- block id -> (m tile, n tile): per-XCD contiguous ranges, N fastest
  const int nblk = mtiles * ntiles;
  int id = blockIdx.x;
  if (nblk >= 2 * NUM_XCD && nblk % NUM_XCD == 0) id = (id % NUM_XCD) * (nblk / NUM_XCD) + id / NUM_XCD;
  const int mt = id / ntiles, nt = id - mt * ntiles;
  const int bm = mt * BM, bn = nt * BN;

  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave % WM, wn = wave / WM;
  const int c = t % CPR;  // this thread's chunk column

  // ---- per-thread A gather state
  int arow[AL], rowb[AL], iy0[AL], ix0[AL];
  bool aval[AL];
#pragma unroll
  for (int i = 0; i < AL; i++) {
    int idx = t + i * NT;
    arow[i] = idx / CPR;
    int m = bm + arow[i];
    aval[i] = idx < BM * CPR && m < M;
    int mm = aval[i] ? m : 0;
    if (KONE) {
      rowb[i] = mm;
      iy0[i] = ix0[i] = 0;
    } else {
      int HWo = y.H * y.W;
      int img = mm / HWo, rem = mm - img * HWo;
      int oy = rem / y.W, ox = rem - oy * y.W;
      rowb[i] = img * x.H;
      iy0[i] = oy * cs - cp;
      ix0[i] = ox * cs - cp;
    }
  }
  const int Cin = x.C;
  int kc = 8 * c;               // flat k of this thread's chunk
  int ci = kc % Cin, tap = kc / Cin;
  int ky = tap / ksz, kx = tap - ky * ksz;

  f16x8 ra[AL], rb[BL];
  const f16x8 zero8 = {0, 0, 0, 0, 0, 0, 0, 0};

  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < AL; i++) {
      ra[i] = zero8;
      if (aval[i] && kc < Ktot) {
        if (KONE) {
          ra[i] = *(const f16x8*)(x.p + (size_t)rowb[i] * x.s + x.o + kc);
        } else {
          int iy = iy0[i] + ky, ix = ix0[i] + kx;
          if (iy >= 0 && iy < x.H && ix >= 0 && ix < x.W)
            ra[i] = *(const f16x8*)(x.p + ((size_t)(rowb[i] + iy) * x.W + ix) * x.s + x.o + ci);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < BL; i++) {
      int idx = t + i * NT;
      int n = bn + idx / CPR;
      int k = k0 + 8 * c;
      rb[i] = zero8;
      if (idx < BN * CPR && n < N && k < Ktot) rb[i] = *(const f16x8*)(w + (size_t)n * Ktot + k);
    }
    // advance this thread's A chunk by one stage
    kc += BK;
    if (!KONE) {
      ci += BK;
      while (ci >= Cin) {
        ci -= Cin;
        if (++kx == ksz) { kx = 0; ky++; }
      }
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < AL; i++)
      if (t + i * NT < BM * CPR) sA[buf][swz<CPR>(arow[i], c)] = ra[i];
#pragma unroll
    for (int i = 0; i < BL; i++) {
      int idx = t + i * NT;
      if (idx < BN * CPR) sB[buf][swz<CPR>(idx / CPR, c)] = rb[i];
    }
  };

  f32x4 acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; i++)
#pragma unroll
    for (int j = 0; j < FM; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nks = (Ktot + BK - 1) / BK;
  gload(0);
  sstore(0);
  __syncthreads();
  const int lr = lane & 15, lg = lane >> 4;
  for (int ks = 0; ks < nks; ks++) {
    const int buf = ks & 1;
    if (ks + 1 < nks) gload((ks + 1) * BK);
#pragma unroll
    for (int s = 0; s < KS; s++) {
      f16x8 fa[FN], fb[FM];
#pragma unroll
      for (int i = 0; i < FN; i++) fa[i] = sB[buf][swz<CPR>(wn * TN + i * 16 + lr, s * 4 + lg)];
#pragma unroll
      for (int j = 0; j < FM; j++) fb[j] = sA[buf][swz<CPR>(wm * TM + j * 16 + lr, s * 4 + lg)];
#pragma unroll
      for (int i = 0; i < FN; i++)
#pragma unroll
        for (int j = 0; j < FM; j++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    if (ks + 1 < nks) sstore(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue: lane holds channels n0..n0+3 of pixel m for every (i, j) fragment
#pragma unroll
  for (int i = 0; i < FN; i++) {
    const int n0 = bn + wn * TN + i * 16 + 4 * lg;
    if (n0 >= N) continue;
    const float b0 = bias[n0], b1 = bias[n0 + 1], b2 = bias[n0 + 2], b3 = bias[n0 + 3];
#pragma unroll
    for (int j = 0; j < FM; j++) {
      const int m = bm + wm * TM + j * 16 + lr;
      if (m >= M) continue;
      float v0 = acc[i][j][0] + b0, v1 = acc[i][j][1] + b1;
      float v2 = acc[i][j][2] + b2, v3 = acc[i][j][3] + b3;
      if (act == 1) { v0 = silu(v0); v1 = silu(v1); v2 = silu(v2); v3 = silu(v3); }
      if (r.p) {
        f16x4 rv = *(const f16x4*)(r.p + (size_t)m * r.s + r.o + n0);
        v0 += (float)rv[0]; v1 += (float)rv[1]; v2 += (float)rv[2]; v3 += (float)rv[3];
      }
      f16x4 o = {(f16)v0, (f16)v1, (f16)v2, (f16)v3};
      *(f16x4*)(y.p + (size_t)m * y.s + y.o + n0) = o;
    }
  }
}

// ------------------------------------------------------------------ tile table
// {BM pixels, BN channels, waves along M, waves along N, BK}
#define YOLO_TILES(X)             \
  X(0, 256, 128, 4, 2, 32)        \
  X(1, 256, 128, 4, 2, 64)        \
  X(2, 128, 128, 2, 2, 64)        \
  X(3, 128, 128, 2, 2, 32)        \
  X(4, 128, 256, 2, 4, 32)        \
  X(5, 256, 64, 4, 1, 64)         \
  X(6, 128, 64, 2, 2, 64)         \
  X(7, 64, 128, 2, 2, 64)         \
  X(8, 64, 64, 2, 2, 64)          \
  X(9, 64, 64, 2, 2, 128)         \
  X(10, 128, 32, 4, 1, 64)        \
  X(11, 64, 32, 2, 2, 128)        \
  X(12, 32, 64, 2, 2, 128)        \
  X(13, 32, 32, 2, 2, 128)        \
  X(14, 128, 16, 4, 1, 64)        \
  X(15, 64, 16, 4, 1, 128)        \
  X(16, 32, 32, 1, 1, 128)        \
  X(17, 64, 64, 1, 1, 128)

static const TileCfg kTiles[] = {
#define X(i, bm, bn, wm, wn, bk) {bm, bn, wm, wn, bk},
    YOLO_TILES(X)
#undef X
};
constexpr int kNumTiles = sizeof(kTiles) / sizeof(kTiles[0]);

int numTileConfigs() { return kNumTiles; }
const TileCfg& tileConfig(int cfg) { return kTiles[cfg]; }

bool tileOk(int cfg, int M, int N, int K) {
  if (cfg < 0 || cfg >= kNumTiles) return false;
  const TileCfg& tc = kTiles[cfg];
  int n16 = (N + 15) / 16 * 16;
  if (tc.BN > 16 && tc.BN / 2 >= n16) return false;      // more than half the N tile idle
  if (tc.BM > 32 && tc.BM / 2 >= M) return false;
  if (tc.BK > 32 && tc.BK / 2 >= K) return false;         // stage mostly padding
  return true;
}

// Default before autotuning: the largest tile whose grid still covers the chip about
// twice (256 CUs) with little N padding, else the one with the most blocks.
int heuristicTile(int M, int N, int K) {
  static const int pref[] = {1, 0, 4, 2, 3, 5, 6, 7, 8, 10, 9, 11, 12, 14, 13, 15, 17, 16};
  int best = -1;
  long bestBlocks = -1;
  for (int cfg : pref) {
    if (!tileOk(cfg, M, N, K)) continue;
    const TileCfg& tc = kTiles[cfg];
    long blocks = (long)((M + tc.BM - 1) / tc.BM) * ((N + tc.BN - 1) / tc.BN);
    long waste = (long)((N + tc.BN - 1) / tc.BN) * tc.BN;
    if (blocks >= 512 && waste * 4 <= (long)N * 5) return cfg;
    if (blocks > bestBlocks) { bestBlocks = blocks; best = cfg; }
  }
  return best < 0 ? 13 : best;
}

template <int BM, int BN, int WM, int WN, int BK>
static void launchTile(bool kone, const View& x, const View& y, const View& r, const f16* w,
                       const float* bias, int k, int s, int p, int act, int M, int N, int Ktot,
                       hipStream_t st) {
  const int mt = (M + BM - 1) / BM, nt = (N + BN - 1) / BN;
  if (kone)
    k_conv_gemm<BM, BN, WM, WN, BK, true><<<mt * nt, 64 * WM * WN, 0, st>>>(x, y, r, w, bias, k, s, p, act, M, N, Ktot, mt, nt);
  else
    k_conv_gemm<BM, BN, WM, WN, BK, false><<<mt * nt, 64 * WM * WN, 0, st>>>(x, y, r, w, bias, k, s, p, act, M, N, Ktot, mt, nt);
}

void launchConvGemm(int cfg, const View& x, const View& y, const View* res, const f16* w,
                    const float* bias, int k, int s, int p, int act, int Bn, hipStream_t st) {
  const int M = Bn * y.H * y.W, N = y.C, Ktot = k * k * x.C;
  const bool kone = (k == 1 && s == 1 && p == 0);
  View r = res ? *res : View{nullptr, 0, 0, 0, 0, 0};
  if (cfg < 0 || cfg >= kNumTiles) cfg = heuristicTile(M, N, Ktot);
  switch (cfg) {
#define X(i, bm, bn, wm, wn, bk) \
    case i: launchTile<bm, bn, wm, wn, bk>(kone, x, y, r, w, bias, k, s, p, act, M, N, Ktot, st); break;
    YOLO_TILES(X)
#undef X
    default: break;
  }
}

// ------------------------------------------------------------------ first conv (Cin = 3)
// 3x3 only (every YOLO stem is 3x3; the loader rejects other sizes).
// One thread per output pixel: the 27 input taps are loaded once into registers and
// reused for every output channel; weights (fp32) and bias sit in LDS and are read as
// wave-uniform broadcasts.  Outputs are written 8 channels (16 bytes) at a time.
constexpr int FIRST_MAX_COUT = 256;

__global__ __launch_bounds__(256) void k_conv_first(View x, View y, const f16* __restrict__ w,
                                                    const float* __restrict__ bias, int cs,
                                                    int cp, int act, int M) {
  __shared__ float sw[FIRST_MAX_COUT * 27];
  __shared__ float sb[FIRST_MAX_COUT];
  const int Cout = y.C, KK = 27;
  for (int i = threadIdx.x; i < Cout * KK; i += blockDim.x) sw[i] = (float)w[i];
  for (int i = threadIdx.x; i < Cout; i += blockDim.x) sb[i] = bias[i];
  __syncthreads();
  const int m = blockIdx.x * blockDim.x + threadIdx.x;
  if (m >= M) return;
  const int HWo = y.H * y.W;
  const int img = m / HWo, rem = m - img * HWo;
  const int oy = rem / y.W, ox = rem - oy * y.W;
  float in[27];
#pragma unroll
  for (int ky = 0; ky < 3; ky++)
#pragma unroll
    for (int kx = 0; kx < 3; kx++) {
      const int iy = oy * cs - cp + ky, ix = ox * cs - cp + kx;
      const bool ok = iy >= 0 && iy < x.H && ix >= 0 && ix < x.W;
      const f16* px = x.p + ((size_t)(img * x.H + (ok ? iy : 0)) * x.W + (ok ? ix : 0)) * x.s + x.o;
#pragma unroll
      for (int q = 0; q < 3; q++) in[(ky * 3 + kx) * 3 + q] = ok ? (float)px[q] : 0.f;
    }
  f16* out = y.p + (size_t)m * y.s + y.o;
  for (int c0 = 0; c0 < Cout; c0 += 8) {
    float a[8];
#pragma unroll
    for (int j = 0; j < 8; j++) a[j] = sb[c0 + j];
#pragma unroll
    for (int wi = 0; wi < 27; wi++) {
      const float v = in[wi];
#pragma unroll
      for (int j = 0; j < 8; j++) a[j] += v * sw[(c0 + j) * KK + wi];
    }
    f16x8 o;
#pragma unroll
    for (int j = 0; j < 8; j++) o[j] = (f16)(act == 1 ? silu(a[j]) : a[j]);
    *(f16x8*)(out + c0) = o;
  }
}

void launchConvFirst(const View& x, const View& y, const f16* w, const float* bias, int s, int p,
                     int act, int Bn, hipStream_t st) {
  const int M = Bn * y.H * y.W;
  k_conv_first<<<(M + 255) / 256, 256, 0, st>>>(x, y, w, bias, s, p, act, M);
}

// ------------------------------------------------------------------ depthwise conv
// One thread per (pixel, 8-channel group); weights were repacked on the host from
// [C][k][k] to [k*k][C] so each tap is one 16-byte load (the reference does the same
// repack, engine/engine.cu:198-209).  fp32 accumulation; optional residual after act.
__global__ __launch_bounds__(256) void k_dwconv(View x, View y, View r, const f16* __restrict__ w,
                                                const float* __restrict__ bias, int ksz, int cs,
                                                int cp, int act, int total) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int cg = y.C >> 3;
  const int g = idx % cg, m = idx / cg;
  const int c = g << 3;
  const int HWo = y.H * y.W;
  const int img = m / HWo, rem = m - img * HWo;
  const int oy = rem / y.W, ox = rem - oy * y.W;
  float a[8];
#pragma unroll
  for (int j = 0; j < 8; j++) a[j] = bias[c + j];
  for (int ky = 0; ky < ksz; ky++) {
    const int iy = oy * cs - cp + ky;
    if (iy < 0 || iy >= x.H) continue;
    for (int kx = 0; kx < ksz; kx++) {
      const int ix = ox * cs - cp + kx;
      if (ix < 0 || ix >= x.W) continue;
      const f16x8 xv = *(const f16x8*)(x.p + ((size_t)(img * x.H + iy) * x.W + ix) * x.s + x.o + c);
      const f16x8 wv = *(const f16x8*)(w + (size_t)(ky * ksz + kx) * y.C + c);
#pragma unroll
      for (int j = 0; j < 8; j++) a[j] += (float)xv[j] * (float)wv[j];
    }
  }
  f16x8 rv = {0, 0, 0, 0, 0, 0, 0, 0};
  if (r.p) rv = *(const f16x8*)(r.p + (size_t)m * r.s + r.o + c);
  f16x8 o;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    float v = act == 1 ? silu(a[j]) : a[j];
    if (r.p) v += (float)rv[j];
    o[j] = (f16)v;
  }
  *(f16x8*)(y.p + (size_t)m * y.s + y.o + c) = o;
}

void launchDwConv(const View& x, const View& y, const View* res, const f16* wt_kkc,
                  const float* bias, int k, int s, int p, int act, int Bn, hipStream_t st) {
  const int total = Bn * y.H * y.W * (y.C / 8);
  View r = res ? *res : View{nullptr, 0, 0, 0, 0, 0};
  k_dwconv<<<(total + 255) / 256, 256, 0, st>>>(x, y, r, wt_kkc, bias, k, s, p, act, total);
}

}  // namespace yolo
