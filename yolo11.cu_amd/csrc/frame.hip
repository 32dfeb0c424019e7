// Frame pre/post-processing kernels: letterbox, DFL decode, NMS, mask assembly.
// Built with -ffp-contract=off so every fp32 expression rounds exactly as written; the
// CPU oracle evaluates the same expressions in the same order and NMS decisions
// (inter/union > thr) are then reproducible bit for bit.
#include "engine.hpp"

namespace yolo {

typedef f16 f16x8 __attribute__((ext_vector_type(8)));

// ------------------------------------------------------------------ letterbox
// BGR u8 HWC (sh x sw) -> RGB fp16 NHWC (dh x dw), /255, pad 114, bilinear with the
// half-pixel map src = (dst + 0.5)/scale - 0.5 and replicate-clamped edges
// (k_preprocess, engine/engine.cu:966-998).  One thread per destination pixel.
__global__ __launch_bounds__(256) void k_letterbox(const uint8_t* __restrict__ src, int sh, int sw,
                                                   f16* __restrict__ dst, int dh, int dw, float scale,
                                                   int top, int left, int nh, int nw) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= dh * dw) return;
  const int x = idx % dw, y = idx / dw;
  float r, g, b;
  if (y < top || y >= top + nh || x < left || x >= left + nw) {
    r = g = b = 114.f;
  } else {
    const float fy = ((float)(y - top) + 0.5f) / scale - 0.5f;
    const float fx = ((float)(x - left) + 0.5f) / scale - 0.5f;
    int y0 = (int)floorf(fy), x0 = (int)floorf(fx);
    const float wy = fy - (float)y0, wx = fx - (float)x0;
    const int y1 = min(max(y0 + 1, 0), sh - 1), x1 = min(max(x0 + 1, 0), sw - 1);
    y0 = min(max(y0, 0), sh - 1);
    x0 = min(max(x0, 0), sw - 1);
    const uint8_t* p00 = src + ((size_t)y0 * sw + x0) * 3;
    const uint8_t* p01 = src + ((size_t)y0 * sw + x1) * 3;
    const uint8_t* p10 = src + ((size_t)y1 * sw + x0) * 3;
    const uint8_t* p11 = src + ((size_t)y1 * sw + x1) * 3;
    const float w00 = (1.f - wy) * (1.f - wx), w01 = (1.f - wy) * wx;
    const float w10 = wy * (1.f - wx), w11 = wy * wx;
    b = (float)p00[0] * w00 + (float)p01[0] * w01 + (float)p10[0] * w10 + (float)p11[0] * w11;
    g = (float)p00[1] * w00 + (float)p01[1] * w01 + (float)p10[1] * w10 + (float)p11[1] * w11;
    r = (float)p00[2] * w00 + (float)p01[2] * w01 + (float)p10[2] * w10 + (float)p11[2] * w11;
  }
  f16* o = dst + (size_t)idx * 3;
  o[0] = (f16)(r / 255.f);
  o[1] = (f16)(g / 255.f);
  o[2] = (f16)(b / 255.f);
}

void launchPreprocess(const uint8_t* src, int sh, int sw, f16* dst, int dh, int dw, float scale,
                      int top, int left, int nh, int nw, hipStream_t st) {
  k_letterbox<<<(dh * dw + 255) / 256, 256, 0, st>>>(src, sh, sw, dst, dh, dw, scale, top, left, nh, nw);
}

// ------------------------------------------------------------------ decode
// One thread per anchor over all levels of all images (one launch instead of one per
// level).  Per anchor (k_decode, engine/engine.cu:844-906): first-max argmax over the nc
// real classes (pad logits excluded), score = sigmoid(best), keep if score >= conf, DFL
// expectation per side, xyxy = (x + 0.5 -+ d) * stride.  Instead of an atomic slot
// counter, every anchor owns slot `anchor` of the candidate array and writes its score
// (or -1) to keys[anchor]; NMS compacts in anchor order, so results do not depend on
// thread scheduling.
__global__ __launch_bounds__(256) void k_decode(DecodeArgs a, float* __restrict__ cand,
                                                float* __restrict__ keys,
                                                const PostParams* __restrict__ prm, int total,
                                                int cstride) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int img = idx / a.A, an = idx - img * a.A;
  int lv = 0;
  if (a.nlev > 1 && an >= a.lv[1].base) lv = 1;
  if (a.nlev > 2 && an >= a.lv[2].base) lv = 2;
  const DecodeLevel& L = a.lv[lv];
  const int local = an - L.base;
  const int yy = local / L.W, xx = local - yy * L.W;
  const size_t pix = (size_t)img * L.H * L.W + local;

  const f16* cp = L.cls.p + pix * L.cls.s + L.cls.o;
  float best = -INFINITY;
  int bcls = 0;
  for (int c0 = 0; c0 < L.cls.C; c0 += 8) {
    const f16x8 v = *(const f16x8*)(cp + c0);
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const float f = (float)v[j];
      if (c0 + j < a.nc && f > best) { best = f; bcls = c0 + j; }
    }
  }
  const float score = 1.f / (1.f + expf(-best));
  const bool keep = score >= prm->conf;
  keys[idx] = keep ? score : -1.f;
  if (!keep) return;

  const f16* bp = L.box.p + pix * L.box.s + L.box.o;
  float d[4];
#pragma unroll
  for (int side = 0; side < 4; side++) {
    const f16x8 v0 = *(const f16x8*)(bp + side * 16), v1 = *(const f16x8*)(bp + side * 16 + 8);
    float l[16];
#pragma unroll
    for (int j = 0; j < 8; j++) { l[j] = (float)v0[j]; l[j + 8] = (float)v1[j]; }
    float mx = l[0];
#pragma unroll
    for (int j = 1; j < 16; j++) mx = fmaxf(mx, l[j]);
    float sum = 0.f, e = 0.f;
#pragma unroll
    for (int j = 0; j < 16; j++) {
      const float p = expf(l[j] - mx);
      sum = sum + p;
      e = e + p * (float)j;
    }
    d[side] = e / sum;
  }
  const float cx = (float)xx + 0.5f, cy = (float)yy + 0.5f, st = (float)L.stride;
  float* o = cand + (size_t)idx * cstride;
  o[0] = (cx - d[0]) * st;
  o[1] = (cy - d[1]) * st;
  o[2] = (cx + d[2]) * st;
  o[3] = (cy + d[3]) * st;
  o[4] = score;
  o[5] = (float)bcls;
  if (a.nm > 0) {
    const f16* mp = L.coef.p + pix * L.coef.s + L.coef.o;
    for (int c0 = 0; c0 < a.nm; c0 += 8) {
      const f16x8 v = *(const f16x8*)(mp + c0);
#pragma unroll
      for (int j = 0; j < 8; j++) o[6 + c0 + j] = (float)v[j];
    }
  }
}

void launchDecode(const DecodeArgs& a, float* cand, float* keys, const PostParams* prm, int Bn,
                  hipStream_t st) {
  const int total = Bn * a.A;
  k_decode<<<(total + 255) / 256, 256, 0, st>>>(a, cand, keys, prm, total, 6 + a.nm);
}

// ------------------------------------------------------------------ NMS
// One block (16 waves) per image.
//  1. compaction: anchors whose key >= 0, in anchor order (wave ballots + block prefix)
//  2. ranking by the total order (score desc, anchor asc) packed in one u64 key; each
//     candidate's rank is the number of larger keys; the top NMS_CAP land in LDS sorted
//  3. greedy suppression (k_nms semantics, engine/engine.cu:1091-1109: same class only,
//     inter/union > thr with a union > 0 guard) resolved 64 candidates at a time: wave 0
//     builds the 64x64 in-block suppression rows and walks them with readlane, then the
//     whole block strikes later candidates that overlap the block's survivors.  This
//     gives exactly the sequential greedy result with two barriers per 64 candidates
//     instead of one per candidate.
constexpr int NMS_THREADS = 1024;

__device__ __forceinline__ bool suppresses(float4 a, float4 b, float thr) {
  const float xx1 = fmaxf(a.x, b.x), yy1 = fmaxf(a.y, b.y);
  const float xx2 = fminf(a.z, b.z), yy2 = fminf(a.w, b.w);
  const float w = fmaxf(0.f, xx2 - xx1), h = fmaxf(0.f, yy2 - yy1);
  const float inter = w * h;
  const float aarea = (a.z - a.x) * (a.w - a.y);
  const float barea = (b.z - b.x) * (b.w - b.y);
  const float ua = aarea + barea - inter;
  return ua > 0.f && inter / ua > thr;
}

__device__ __forceinline__ unsigned long long packKey(float score, int anchor) {
  return ((unsigned long long)__float_as_uint(score) << 32) | (unsigned)(0xFFFFFFFFu - (unsigned)anchor);
}

__global__ __launch_bounds__(NMS_THREADS) void k_nms(const float* __restrict__ cand,
                                                     const float* __restrict__ keys, int A,
                                                     int cstride, float* __restrict__ out,
                                                     int* __restrict__ outidx, int* __restrict__ outcnt,
                                                     int* __restrict__ rawcnt,
                                                     unsigned long long* __restrict__ scratch,
                                                     const PostParams* __restrict__ prm) {
  __shared__ unsigned long long skey[NMS_CAP];
  __shared__ float4 sbox[NMS_CAP];
  __shared__ short scls[NMS_CAP];
  __shared__ unsigned removed[NMS_CAP / 32];
  __shared__ int wcnt[NMS_THREADS / 64];
  __shared__ unsigned long long keptmask;
  __shared__ int nout;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int img = blockIdx.x;
  const float* kimg = keys + (size_t)img * A;
  const float* cimg = cand + (size_t)img * A * cstride;
  unsigned long long* lst = scratch + (size_t)img * A;
  const float thr = prm->iou;
  const int maxdet = min(prm->max_det, MAX_OUT);

  // 1. compaction in anchor order
  int n = 0;
  for (int base = 0; base < A; base += NMS_THREADS) {
    const int an = base + tid;
    const float kv = an < A ? kimg[an] : -1.f;
    const bool f = kv >= 0.f;
    const unsigned long long bal = __ballot(f);
    const int pre = __popcll(bal & ((1ull << lane) - 1ull));
    if (lane == 0) wcnt[wave] = __popcll(bal);
    __syncthreads();
    int off = n, tot = 0;
    for (int w = 0; w < NMS_THREADS / 64; w++) {
      if (w < wave) off += wcnt[w];
      tot += wcnt[w];
    }
    if (f) lst[off + pre] = packKey(kv, an);
    n += tot;
    __syncthreads();
  }
  const int m = min(n, NMS_CAP);

  // 2. rank: position = number of strictly larger keys (keys are unique)
  for (int i = tid; i < n; i += NMS_THREADS) {
    const unsigned long long ki = lst[i];
    int rank = 0;
    for (int j = 0; j < n; j++) rank += lst[j] > ki;
    if (rank < NMS_CAP) skey[rank] = ki;
  }
  for (int i = tid; i < NMS_CAP / 32; i += NMS_THREADS) removed[i] = 0u;
  if (tid == 0) nout = 0;
  __syncthreads();
  for (int r = tid; r < m; r += NMS_THREADS) {
    const int an = (int)(0xFFFFFFFFu - (unsigned)(skey[r] & 0xFFFFFFFFull));
    const float* rec = cimg + (size_t)an * cstride;
    sbox[r] = make_float4(rec[0], rec[1], rec[2], rec[3]);
    scls[r] = (short)rec[5];
  }
  __syncthreads();

  // 3. greedy, 64 candidates per step
  for (int cb = 0; cb * 64 < m; cb++) {
    if (nout >= maxdet) break;
    if (wave == 0) {
      const int i = cb * 64 + lane;
      unsigned long long row = 0ull;
      if (i < m) {
        const float4 bi = sbox[i];
        const short ci = scls[i];
        for (int jj = lane + 1; jj < 64; jj++) {
          const int j = cb * 64 + jj;
          if (j < m && scls[j] == ci && suppresses(bi, sbox[j], thr)) row |= 1ull << jj;
        }
      }
      const unsigned long long valid = (m - cb * 64) >= 64 ? ~0ull : ((1ull << (m - cb * 64)) - 1ull);
      unsigned long long alive =
          ~(((unsigned long long)removed[2 * cb + 1] << 32) | removed[2 * cb]) & valid;
      for (int tt = 0; tt < 64; tt++) {
        if ((alive >> tt) & 1ull) {
          const unsigned lo = __builtin_amdgcn_readlane((unsigned)row, tt);
          const unsigned hi = __builtin_amdgcn_readlane((unsigned)(row >> 32), tt);
          alive &= ~(((unsigned long long)hi << 32) | lo);
        }
      }
      const int slot = nout + __popcll(alive & ((1ull << lane) - 1ull));
      if (((alive >> lane) & 1ull) && slot < maxdet) {
        const int an = (int)(0xFFFFFFFFu - (unsigned)(skey[i] & 0xFFFFFFFFull));
        const float4 bi = sbox[i];
        float* d = out + ((size_t)img * MAX_OUT + slot) * 6;
        d[0] = bi.x; d[1] = bi.y; d[2] = bi.z; d[3] = bi.w;
        d[4] = __uint_as_float((unsigned)(skey[i] >> 32));
        d[5] = (float)scls[i];
        outidx[img * MAX_OUT + slot] = an;
      }
      if (lane == 0) {
        keptmask = alive;
        nout = nout + __popcll(alive);
      }
    }
    __syncthreads();
    const unsigned long long km = keptmask;
    if (km) {
      for (int j = (cb + 1) * 64 + tid; j < m; j += NMS_THREADS) {
        if ((removed[j >> 5] >> (j & 31)) & 1u) continue;
        const float4 bj = sbox[j];
        const short cj = scls[j];
        unsigned long long bits = km;
        while (bits) {
          const int tt = __ffsll((long long)bits) - 1;
          bits &= bits - 1ull;
          const int i = cb * 64 + tt;
          if (scls[i] == cj && suppresses(sbox[i], bj, thr)) {
            atomicOr(&removed[j >> 5], 1u << (j & 31));
            break;
          }
        }
      }
    }
    __syncthreads();
  }
  if (tid == 0) {
    outcnt[img] = min(nout, maxdet);
    rawcnt[img] = n;
  }
}

size_t nmsScratchBytes(int A) { return (size_t)A * sizeof(unsigned long long); }

void launchNms(const float* cand, const float* keys, int A, int cstride, float* out, int* outidx,
               int* outcnt, int* rawcnt, unsigned long long* scratch, const PostParams* prm,
               int Bn, hipStream_t st) {
  k_nms<<<Bn, NMS_THREADS, 0, st>>>(cand, keys, A, cstride, out, outidx, outcnt, rawcnt, scratch, prm);
}

// ------------------------------------------------------------------ masks
// Survivor masks at proto resolution (k_mask_assemble, engine/engine.cu:1125-1158):
// logit = coef . proto (fp32), pixel kept iff inside the box scaled to proto resolution
// (half-open float compares) and logit > 0.  One block per (survivor slot, image); slots
// past the image's count exit, so the fixed grid can live in a graph.
__global__ __launch_bounds__(256) void k_masks(View proto, const float* __restrict__ cand, int cstride,
                                               int A, int nm, const int* __restrict__ outidx,
                                               const int* __restrict__ outcnt,
                                               const float* __restrict__ outdets,
                                               uint8_t* __restrict__ masks, float rx, float ry) {
  const int d = blockIdx.x, img = blockIdx.y;
  if (d >= outcnt[img]) return;
  __shared__ float co[64];
  const int an = outidx[img * MAX_OUT + d];
  const float* cf = cand + ((size_t)img * A + an) * cstride + 6;
  if ((int)threadIdx.x < nm) co[threadIdx.x] = cf[threadIdx.x];
  __syncthreads();
  const float* det = outdets + ((size_t)img * MAX_OUT + d) * 6;
  const float bx1 = det[0] * rx, by1 = det[1] * ry, bx2 = det[2] * rx, by2 = det[3] * ry;
  const int Ph = proto.H, Pw = proto.W;
  uint8_t* mo = masks + ((size_t)img * MAX_OUT + d) * Ph * Pw;
  const f16* pimg = proto.p + (size_t)img * Ph * Pw * proto.s + proto.o;
  for (int p = threadIdx.x; p < Ph * Pw; p += blockDim.x) {
    const int px = p % Pw, py = p / Pw;
    const f16* pp = pimg + (size_t)p * proto.s;
    float acc = 0.f;
    for (int c0 = 0; c0 < nm; c0 += 8) {
      const f16x8 v = *(const f16x8*)(pp + c0);
#pragma unroll
      for (int j = 0; j < 8; j++) acc = acc + co[c0 + j] * (float)v[j];
    }
    const bool in = (float)px >= bx1 && (float)px < bx2 && (float)py >= by1 && (float)py < by2;
    mo[p] = (in && acc > 0.f) ? 1 : 0;
  }
}

void launchMasks(const View& proto, const float* cand, int cstride, int A, int nm,
                 const int* outidx, const int* outcnt, const float* outdets, uint8_t* masks,
                 float rx, float ry, int Bn, hipStream_t st) {
  k_masks<<<dim3(MAX_OUT, Bn), 256, 0, st>>>(proto, cand, cstride, A, nm, outidx, outcnt, outdets,
                                            masks, rx, ry);
}

}  // namespace yolo
