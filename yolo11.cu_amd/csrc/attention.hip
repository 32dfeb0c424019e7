// C2PSA attention for gfx950: one fused kernel per ATTN op.
//
// Semantics (export/export.py:492-500; the reference runs it as 2*heads+2 launches per
// image through its GEMM kernel plus a softmax and a V-transpose kernel,
// engine/engine.cu:1363-1397):
//   qkv view [B][N][heads * (2kd + hd)], per head [q (kd) | k (kd) | v (hd)]
//   out[b][n][h*hd + c] = sum_j softmax_j(q_n . k_j * kd^-1/2) * v_j[c]
//
// Design: one block per (image, head, 64-query group); a block of 4 waves owns 64 queries
// and walks the keys in chunks of 64, flash-style, so the N x N score matrix never exists in
// memory.  Small N (every key fits LDS) stages all keys at once.  Every query group of an
// (image, head) reads the same K and V, so the blocks are numbered to put the groups of one
// (image, head) on one XCD (dispatch is round-robin over the 8 XCDs, each with its own L2):
// the groups after the first read K and V from that L2 instead of HBM.
//  * Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_16x16x32_f16 (kd = 32 is
//    one MFMA K step): each lane then holds 16 scores of ONE query, so the online-softmax
//    max needs only a 4-lane-group exchange and the running sum stays lane-local.
//  * O^T = V^T P^T, again one MFMA per 32 keys per 16 channels.  The probabilities never
//    leave registers: the k-index assignment of the P operand is simply the one the score
//    tiles already have, and V^T is read from LDS with the same assignment (the MFMA sum
//    over k does not depend on how k is distributed, only that A and B agree).
//  * exp is exp2 with log2(e) folded into the score scale; fp32 statistics, fp16 P and V,
//    fp32 accumulation.
#include "engine.hpp"
#include "viewcopy.hpp"

namespace yolo {

typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int AQ = 64;      // queries per block
constexpr int AK = 64;      // keys per chunk
constexpr int VT_PITCH = 72;  // halves per V^T row in LDS (64 keys + 8 pad, breaks bank aliasing)

__device__ __forceinline__ int kswz(int row, int c) { return row * 4 + (c ^ ((row >> 1) & 3)); }

// WHOLE: every key of the (image, head) is staged in LDS once (dynamic LDS, N <= ATT_WHOLE_MAX)
// with all global loads in flight together, and the chunk loop then runs without barriers;
// otherwise keys stream through a 64-key buffer, one barrier pair per chunk.
// KS (WHOLE only): the key chunks of a query group are split over KS wave groups (chunks
// kp, kp + KS, ...), each with its own online-softmax state; at the end the groups' (max,
// sum, O) partials are merged through LDS.  Small grids (batch 1) use KS = 4, so four
// waves share what one wave would walk alone.
constexpr int ATT_WHOLE_MAX = 512;
constexpr size_t ATT_WHOLE_LDS = 128 * 1024;   // dynamic LDS opt-in set by attentionInit()
static bool attWholeOk = false;                 // the opt-in succeeded

constexpr int NUM_XCD = 8;

// Linear block b -> work item: the j-th block of XCD class x = b % 8 takes item
// x * q + min(x, r) + j (q = n / 8, r = n % 8), a bijection on [0, n) that gives each XCD a
// contiguous range of items.
__device__ __forceinline__ int xcdItem(int b, int n) {
  const int x = b % NUM_XCD, j = b / NUM_XCD, q = n / NUM_XCD, r = n % NUM_XCD;
  return x * q + min(x, r) + j;
}

// Blocks [0, natt) are the attention's; any after them run the channel copies in `riders`.
template <int HD, bool WHOLE, int KS>
__global__ __launch_bounds__(256 * KS) void k_attention(View qkv, View y, int N, int heads, float scale_log2,
                                                        int natt, const CopyLaunch riders) {
  constexpr int KD = 32;
  constexpr int CT = HD / 16;  // channel tiles of the output
  constexpr int NT = 256 * KS;
  static_assert(WHOLE || KS == 1, "key splits need every key in LDS");
  extern __shared__ f16x8 dyn[];
  __shared__ f16x8 sKs[WHOLE ? 1 : AK * 4];
  __shared__ f16 sVts[WHOLE ? 1 : HD * VT_PITCH];

  if ((int)blockIdx.x >= natt) {   // block-uniform: a carried copy, no LDS, no barrier
    runCopyBlock(riders, (int)blockIdx.x - natt);
    return;
  }
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int qw = wave & 3, kp = wave >> 2;   // query group, key part
  const int lr = lane & 15, lg = lane >> 4;
  // items are (image, head, query group), query group fastest
  const int nq = (N + AQ - 1) / AQ, items = natt;
  const int item = items >= 2 * NUM_XCD ? xcdItem((int)blockIdx.x, items) : (int)blockIdx.x;
  const int qgrp = item % nq, h = (item / nq) % heads, img = item / (nq * heads);
  const int per = 2 * KD + HD;
  const int qoff = qkv.o + h * per;
  const size_t imgbase = (size_t)img * N;  // token index base of this image
  const int nchunk = (N + AK - 1) / AK;
  const int NP = nchunk * AK;
  const int vpitch = WHOLE ? NP + 8 : VT_PITCH;
  f16x8* sK = WHOLE ? dyn : sKs;
  f16* sVt = WHOLE ? (f16*)(dyn + NP * 4) : sVts;

  // stage keys [k0, k0 + cnt) into LDS rows kbase.. (K as 4 swizzled 16-byte chunks, V^T)
  auto stage = [&](int k0, int cnt, int kbase) {
    for (int i = t; i < cnt * 4; i += NT) {
      const int key = i >> 2, c = i & 3;
      f16x8 kv = {0, 0, 0, 0, 0, 0, 0, 0};
      if (k0 + key < N) kv = *(const f16x8*)(qkv.p + (imgbase + k0 + key) * qkv.s + qoff + KD + 8 * c);
      sK[kswz(kbase + key, c)] = kv;
    }
    for (int i = t; i < cnt * (HD / 8); i += NT) {
      const int key = i / (HD / 8), g = i - key * (HD / 8);
      f16x8 vv = {0, 0, 0, 0, 0, 0, 0, 0};
      if (k0 + key < N) vv = *(const f16x8*)(qkv.p + (imgbase + k0 + key) * qkv.s + qoff + 2 * KD + 8 * g);
#pragma unroll
      for (int j = 0; j < 8; j++) sVt[(8 * g + j) * vpitch + kbase + key] = vv[j];
    }
  };

  // Q fragment: query lr of this wave, dims 8*lg .. 8*lg+7 (MFMA B operand)
  const int q = qgrp * AQ + qw * 16 + lr;
  f16x8 fq = {0, 0, 0, 0, 0, 0, 0, 0};
  if (q < N) fq = *(const f16x8*)(qkv.p + (imgbase + q) * qkv.s + qoff + 8 * lg);

  float mrun = -INFINITY, lrun = 0.f;
  f32x4 oacc[CT];
#pragma unroll
  for (int i = 0; i < CT; i++) oacc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (WHOLE) {
    // every key at once, all global loads issued before the first LDS store.  V goes in as
    // items of 8 keys x 8 channels: 8 row loads, an in-register 8x8 transpose, and 8
    // 16-byte V^T row stores
    constexpr int KIT = (ATT_WHOLE_MAX * 4 + NT - 1) / NT;
    constexpr int VIT = (ATT_WHOLE_MAX / 8 * (HD / 8) + NT - 1) / NT;
    f16x8 kv[KIT], vv[VIT][8];
#pragma unroll
    for (int u = 0; u < KIT; u++) {
      const int i = t + NT * u, key = i >> 2;
      kv[u] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
      if (key < N) kv[u] = *(const f16x8*)(qkv.p + (imgbase + key) * qkv.s + qoff + KD + 8 * (i & 3));
    }
#pragma unroll
    for (int u = 0; u < VIT; u++) {
      const int i = t + NT * u, kb = i / (HD / 8), g = i - kb * (HD / 8);
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const int key = 8 * kb + j;
        vv[u][j] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
        if (key < N) vv[u][j] = *(const f16x8*)(qkv.p + (imgbase + key) * qkv.s + qoff + 2 * KD + 8 * g);
      }
    }
#pragma unroll
    for (int u = 0; u < KIT; u++) {
      const int i = t + NT * u, key = i >> 2;
      if (key < NP) sK[kswz(key, i & 3)] = kv[u];
    }
#pragma unroll
    for (int u = 0; u < VIT; u++) {
      const int i = t + NT * u, kb = i / (HD / 8), g = i - kb * (HD / 8);
      if (8 * kb < NP) {
#pragma unroll
        for (int c = 0; c < 8; c++) {
          f16x8 row;
#pragma unroll
          for (int j = 0; j < 8; j++) row[j] = vv[u][j][c];
          *(f16x8*)(sVt + (8 * g + c) * vpitch + 8 * kb) = row;
        }
      }
    }
    __syncthreads();
  }
#pragma unroll 2
  for (int ch = kp; ch < nchunk; ch += KS) {
    const int k0 = ch * AK;
    const int kb = WHOLE ? k0 : 0;   // LDS row of this chunk's first key
    if (!WHOLE) {
      stage(k0, AK, 0);
      __syncthreads();
    }

    // ---- S^T tiles: lane holds scores of query lr for keys kt*16 + 4*lg + r
    float s[4][4];
    float cmax = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 4; kt++) {
      f16x8 fk = sK[kswz(kb + kt * 16 + lr, lg)];
      f32x4 z = __builtin_amdgcn_mfma_f32_16x16x32_f16(fk, fq, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int key = k0 + kt * 16 + 4 * lg + r;
        s[kt][r] = key < N ? z[r] * scale_log2 : -INFINITY;
        cmax = fmaxf(cmax, s[kt][r]);
      }
    }
    cmax = fmaxf(cmax, __shfl_xor(cmax, 16));
    cmax = fmaxf(cmax, __shfl_xor(cmax, 32));
    const float mnew = fmaxf(mrun, cmax);
    const float alpha = exp2f(mrun - mnew);
    mrun = mnew;
    float psum = 0.f;
#pragma unroll
    for (int kt = 0; kt < 4; kt++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        s[kt][r] = exp2f(s[kt][r] - mnew);
        psum += s[kt][r];
      }
    lrun = lrun * alpha + psum;
#pragma unroll
    for (int i = 0; i < CT; i++) oacc[i] *= alpha;

    // ---- O^T += V^T P^T, 32 keys per MFMA: element e<4 -> key 4lg+e, e>=4 -> 16+4lg+e-4
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
      f16x8 fp;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        fp[e] = (f16)s[2 * hh][e];
        fp[4 + e] = (f16)s[2 * hh + 1][e];
      }
#pragma unroll
      for (int i = 0; i < CT; i++) {
        const f16* vrow = sVt + (i * 16 + lr) * vpitch + kb + hh * 32 + 4 * lg;
        const f16x4 v0 = *(const f16x4*)(vrow);
        const f16x4 v1 = *(const f16x4*)(vrow + 16);
        f16x8 fv = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
        oacc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fv, fp, oacc[i], 0, 0, 0);
      }
    }
    if (!WHOLE) __syncthreads();
  }

  if constexpr (KS > 1) {
    // merge the key parts: parts 1.. park (max, partial sum, O) in the (now free) key
    // storage, part 0 rescales everything to the common max and adds
    constexpr int REC = 2 + 4 * CT;   // floats per lane
    float* park = reinterpret_cast<float*>(dyn);
    __syncthreads();
    if (kp > 0) {
      float* rec = park + ((size_t)((kp - 1) * 4 + qw) * 64 + lane) * REC;
      rec[0] = mrun;
      rec[1] = lrun;
#pragma unroll
      for (int i = 0; i < CT; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) rec[2 + 4 * i + r] = oacc[i][r];
    }
    __syncthreads();
    if (kp > 0) return;
    float mt = mrun;
#pragma unroll
    for (int pp = 1; pp < KS; pp++) mt = fmaxf(mt, park[((size_t)((pp - 1) * 4 + qw) * 64 + lane) * REC]);
    const float a0 = exp2f(mrun - mt);
    lrun *= a0;
#pragma unroll
    for (int i = 0; i < CT; i++) oacc[i] *= a0;
#pragma unroll
    for (int pp = 1; pp < KS; pp++) {
      const float* rec = park + ((size_t)((pp - 1) * 4 + qw) * 64 + lane) * REC;
      const float ap = exp2f(rec[0] - mt);
      lrun += rec[1] * ap;
#pragma unroll
      for (int i = 0; i < CT; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) oacc[i][r] += rec[2 + 4 * i + r] * ap;
    }
  }

  lrun += __shfl_xor(lrun, 16);
  lrun += __shfl_xor(lrun, 32);
  if (q >= N) return;
  const float inv = 1.f / lrun;
  f16* out = y.p + (imgbase + q) * y.s + y.o + h * HD;
#pragma unroll
  for (int i = 0; i < CT; i++) {
    f16x4 o = {(f16)(oacc[i][0] * inv), (f16)(oacc[i][1] * inv), (f16)(oacc[i][2] * inv),
               (f16)(oacc[i][3] * inv)};
    *(f16x4*)(out + i * 16 + 4 * lg) = o;
  }
}

// dynamic LDS of a whole-key launch: the staged keys, or the merge records if larger
template <int HD>
static size_t attWholeLds(int N, int KS) {
  const int NP = (N + AK - 1) / AK * AK;
  const size_t stage = (size_t)NP * 4 * sizeof(f16x8) + (size_t)HD * (NP + 8) * sizeof(f16);
  const size_t merge = KS > 1 ? (size_t)(KS - 1) * 4 * 64 * (2 + HD / 4) * sizeof(float) : 0;
  return stage > merge ? stage : merge;
}

template <int HD>
static void launchAttn(const View& qkv, const View& y, int N, int heads, float sl2, int Bn, hipStream_t st,
                       const View* xs, const View* ys, int ncopy) {
  const int nq = (N + AQ - 1) / AQ;
  const int natt = nq * heads * Bn;
  // key splits while one image's grid leaves most CUs idle.  Decided per image, not per
  // launch, so an image's result does not depend on the batch it runs in (the splits change
  // the softmax merge order).
  const long blocks = (long)nq * heads;
  const int KS = blocks <= 128 ? 4 : blocks <= 512 ? 2 : 1;
  const bool whole = attWholeOk && N <= ATT_WHOLE_MAX && attWholeLds<HD>(N, KS) <= ATT_WHOLE_LDS;
  // carried copies go after the attention's blocks, into the CUs its last wave leaves idle
  int ncb = 0;
  const CopyLaunch L = copyLaunch(xs, ys, ncopy, Bn, whole ? 256 * KS : 256, &ncb);
  const dim3 grid(natt + ncb);
  if (whole) {
    const size_t lds = attWholeLds<HD>(N, KS);
    if (KS == 4) k_attention<HD, true, 4><<<grid, 256 * 4, lds, st>>>(qkv, y, N, heads, sl2, natt, L);
    else if (KS == 2) k_attention<HD, true, 2><<<grid, 256 * 2, lds, st>>>(qkv, y, N, heads, sl2, natt, L);
    else k_attention<HD, true, 1><<<grid, 256, lds, st>>>(qkv, y, N, heads, sl2, natt, L);
  } else {
    k_attention<HD, false, 1><<<grid, 256, 0, st>>>(qkv, y, N, heads, sl2, natt, L);
  }
}

// Whole-key kernels use more than the default 64 KiB of dynamic LDS; opt them in once per
// process (a function attribute, not a stream operation).
void attentionInit() {
  bool ok = true;
#define ATT_ALLOW1(HD, KS)                                                                     \
  ok = ok && hipFuncSetAttribute((const void*)k_attention<HD, true, KS>,                       \
                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)ATT_WHOLE_LDS) == hipSuccess;
#define ATT_ALLOW(HD) ATT_ALLOW1(HD, 1) ATT_ALLOW1(HD, 2) ATT_ALLOW1(HD, 4)
  ATT_ALLOW(16) ATT_ALLOW(32) ATT_ALLOW(48) ATT_ALLOW(64) ATT_ALLOW(80) ATT_ALLOW(96) ATT_ALLOW(112) ATT_ALLOW(128)
#undef ATT_ALLOW
#undef ATT_ALLOW1
  (void)hipGetLastError();
  attWholeOk = ok;
}

void launchAttention(const View& qkv, const View& y, int heads, int kd, int hd, int Bn,
                     hipStream_t st, const View* xs, const View* ys, int ncopy) {
  (void)kd;  // the loader accepts kd == 32 only
  const int N = qkv.H * qkv.W;
  const float scale_log2 = (1.0f / sqrtf(32.0f)) * 1.4426950408889634f;
  switch (hd) {
    case 16: launchAttn<16>(qkv, y, N, heads, scale_log2, Bn, st, xs, ys, ncopy); break;
    case 32: launchAttn<32>(qkv, y, N, heads, scale_log2, Bn, st, xs, ys, ncopy); break;
    case 48: launchAttn<48>(qkv, y, N, heads, scale_log2, Bn, st, xs, ys, ncopy); break;
    case 64: launchAttn<64>(qkv, y, N, heads, scale_log2, Bn, st, xs, ys, ncopy); break;
    case 80: launchAttn<80>(qkv, y, N, heads, scale_log2, Bn, st, xs, ys, ncopy); break;
    case 96: launchAttn<96>(qkv, y, N, heads, scale_log2, Bn, st, xs, ys, ncopy); break;
    case 112: launchAttn<112>(qkv, y, N, heads, scale_log2, Bn, st, xs, ys, ncopy); break;
    case 128: launchAttn<128>(qkv, y, N, heads, scale_log2, Bn, st, xs, ys, ncopy); break;
    default: break;
  }
}

}  // namespace yolo
