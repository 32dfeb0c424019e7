// Frame pre/post-processing kernels: letterbox, DFL decode, NMS, mask assembly.
// Built with -ffp-contract=off so every fp32 expression rounds exactly as written; the
// CPU oracle evaluates the same expressions in the same order and NMS decisions
// (inter/union > thr) are then reproducible bit for bit.
#include "boxes.hpp"

namespace yolo {

typedef f16 f16x8 __attribute__((ext_vector_type(8)));

// ------------------------------------------------------------------ letterbox
// Channel c (0 blue, 1 green, 2 red) of source pixel i in layout fmt (PIXEL_BGR: B, G, R;
// PIXEL_RGBX: R, G, B, X).  Both layouts give the same values, so results do not depend on it.
__device__ __forceinline__ float srcChan(const uint8_t* __restrict__ src, size_t i, int fmt, int c) {
  return fmt == PIXEL_RGBX ? (float)src[i * 4 + (2 - c)] : (float)src[i * 3 + c];
}

// BGR (or RGBX) u8 HWC (sh x sw) -> RGB fp16 NHWC (dh x dw), /255, pad 114, bilinear with
// the half-pixel map src = (dst + 0.5)/scale - 0.5 and replicate-clamped edges
// (k_preprocess, engine/engine.cu:966-998).  One thread per destination pixel.
// One letterbox output pixel: bilinear sample of the scaled image, pad 114 outside it, BGR ->
// RGB, /255.
__device__ __forceinline__ void letterboxPixel(const uint8_t* __restrict__ src, int sh, int sw, int fmt,
                                               f16* __restrict__ dst, int dw, float scale, int top,
                                               int left, int nh, int nw, int idx) {
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
    const size_t i00 = (size_t)y0 * sw + x0, i01 = (size_t)y0 * sw + x1;
    const size_t i10 = (size_t)y1 * sw + x0, i11 = (size_t)y1 * sw + x1;
    const float w00 = (1.f - wy) * (1.f - wx), w01 = (1.f - wy) * wx;
    const float w10 = wy * (1.f - wx), w11 = wy * wx;
    float v[3];
    for (int c = 0; c < 3; c++)
      v[c] = srcChan(src, i00, fmt, c) * w00 + srcChan(src, i01, fmt, c) * w01 +
             srcChan(src, i10, fmt, c) * w10 + srcChan(src, i11, fmt, c) * w11;
    b = v[0];
    g = v[1];
    r = v[2];
  }
  f16* o = dst + (size_t)idx * 3;
  o[0] = (f16)(r / 255.f);
  o[1] = (f16)(g / 255.f);
  o[2] = (f16)(b / 255.f);
}

__global__ __launch_bounds__(256) void k_letterbox(const uint8_t* __restrict__ src, int sh, int sw,
                                                   f16* __restrict__ dst, int dh, int dw, float scale,
                                                   int top, int left, int nh, int nw) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= dh * dw) return;
  letterboxPixel(src, sh, sw, PIXEL_BGR, dst, dw, scale, top, left, nh, nw, idx);
}

// All frames of a batch in one launch (blockIdx.y = slot within the chunk); each slot has its
// own source and geometry, and writes its image of the dh x dw x 3 input batch.
__global__ __launch_bounds__(256) void k_letterbox_batch(LetterboxBatch lb, f16* __restrict__ dst, int dh,
                                                         int dw) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= dh * dw) return;
  const LetterboxSlot& s = lb.slot[blockIdx.y];
  letterboxPixel(s.src, s.sh, s.sw, s.fmt, dst + (size_t)s.index * dh * dw * 3, dw, s.scale, s.top, s.left,
                 s.nh, s.nw, idx);
}

void launchPreprocess(const uint8_t* src, int sh, int sw, f16* dst, int dh, int dw, float scale,
                      int top, int left, int nh, int nw, hipStream_t st) {
  k_letterbox<<<(dh * dw + 255) / 256, 256, 0, st>>>(src, sh, sw, dst, dh, dw, scale, top, left, nh, nw);
}

void launchPreprocessBatch(const LetterboxSlot* slots, int n, f16* dst, int dh, int dw, hipStream_t st) {
  for (int s0 = 0; s0 < n; s0 += LETTERBOX_BATCH) {
    LetterboxBatch lb;
    const int k = n - s0 < LETTERBOX_BATCH ? n - s0 : LETTERBOX_BATCH;
    for (int i = 0; i < k; i++) lb.slot[i] = slots[s0 + i];
    k_letterbox_batch<<<dim3((dh * dw + 255) / 256, k), 256, 0, st>>>(lb, dst, dh, dw);
  }
}

// ------------------------------------------------------------------ classify preprocess
// BGR (or RGBX) u8 HWC (sh x sw) -> RGB fp16 NHWC (S x S), /255: resize the shortest edge to S with
// the antialiased bilinear (triangle) filter of PIL / torchvision, whose support widens by
// the scale when downscaling, then centre-crop S x S (k_preprocess_cls,
// engine/engine.cu:1000-1034; the host gives the resized size rh x rw and the crop offsets).
// One thread per destination pixel; the tap weights and sums are evaluated in the
// reference's order so the fp32 result is reproducible bit for bit.
__global__ __launch_bounds__(256) void k_preprocess_cls(const uint8_t* __restrict__ src, int sh, int sw,
                                                        f16* __restrict__ dst, int S, int rh, int rw,
                                                        int top, int left, int fmt) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= S * S) return;
  const int ox = idx % S, oy = idx / S;
  const float fy = (float)sh / (float)rh, fx = (float)sw / (float)rw;   // source px per resized px
  const float ry = fmaxf(fy, 1.f), rx = fmaxf(fx, 1.f);                 // filter radius
  const float cy = ((float)(oy + top) + 0.5f) * fy, cx = ((float)(ox + left) + 0.5f) * fx;
  const int ya = max(0, (int)(cy - ry + 0.5f)), yb = min(sh, (int)(cy + ry + 0.5f));
  const int xa = max(0, (int)(cx - rx + 0.5f)), xb = min(sw, (int)(cx + rx + 0.5f));
  auto tri = [](float d, float r) { return fmaxf(0.f, 1.f - fabsf(d) / r); };
  float ny = 0.f, nx = 0.f;
  for (int i = ya; i < yb; i++) ny += tri((float)i + 0.5f - cy, ry);
  for (int j = xa; j < xb; j++) nx += tri((float)j + 0.5f - cx, rx);
  float sb = 0.f, sg = 0.f, sr = 0.f;
  for (int i = ya; i < yb; i++) {
    const float wy = tri((float)i + 0.5f - cy, ry);
    for (int j = xa; j < xb; j++) {
      const float w = wy * tri((float)j + 0.5f - cx, rx);
      const size_t px = (size_t)i * sw + j;
      sb += w * srcChan(src, px, fmt, 0);
      sg += w * srcChan(src, px, fmt, 1);
      sr += w * srcChan(src, px, fmt, 2);
    }
  }
  const float inv = 1.f / (ny * nx * 255.f);
  // the products are rounded to fp32 before the fp16 conversion: without the barrier the
  // compiler fuses multiply and conversion (v_fma_mixlo_f16, one rounding), which differs
  // from the reference's two roundings near fp16 midpoints
  float vr = sr * inv, vg = sg * inv, vb = sb * inv;
  asm volatile("" : "+v"(vr), "+v"(vg), "+v"(vb));
  f16* o = dst + (size_t)idx * 3;
  o[0] = (f16)vr;
  o[1] = (f16)vg;
  o[2] = (f16)vb;
}

void launchPreprocessCls(const uint8_t* src, int sh, int sw, f16* dst, int S, int rh, int rw, int top,
                         int left, int fmt, hipStream_t st) {
  k_preprocess_cls<<<(S * S + 255) / 256, 256, 0, st>>>(src, sh, sw, dst, S, rh, rw, top, left, fmt);
}

// ------------------------------------------------------------------ decode
// Four lanes per anchor over all levels of all images (one launch instead of one per level).
// Per anchor (k_decode, engine/engine.cu:844-906): first-max argmax over the nc real classes
// (pad logits excluded), score = sigmoid(best), keep if score >= conf, DFL expectation per
// side, xyxy = (x + 0.5 -+ d) * stride.  Lane q of an anchor takes class chunks q, q + 4, ...
// (8 classes each, in increasing order, first max within them) and the four lanes merge
// (value, class) with the lower class winning ties -- the sequential first max; if kept,
// lane q computes the DFL expectation of side q in the sequential order.  Every anchor owns
// record `anchor` of the candidate array; survivors append a packed (score, anchor) key to
// the image's list, which NMS ranks, so results do not depend on thread scheduling.
// grid (blocks of 64 anchors, images): a wave never spans two images, so the survivors of a
// wave are appended to the image's candidate list with one atomic (wave-aggregated).  The
// list order depends on arrival; NMS sorts by key, so results do not.
// OBB (k_decode_obb, engine/engine.cu:908-964): the angle view (channel 0 real) gives
// theta = (sigmoid(t) - 0.25) * pi, the DFL distances are rotated by theta about the anchor
// (dist2rbox), w = l + r, h = t + b, and the record is cx, cy, w, h, score, cls, theta.
constexpr int DEC_ANCHORS = 64;   // anchors per block (4 lanes each)
template <bool OBB>
__global__ __launch_bounds__(4 * DEC_ANCHORS) void k_decode(DecodeArgs a, float* __restrict__ cand,
                                                             unsigned long long* __restrict__ lst,
                                                             int* __restrict__ count,
                                                             const PostParams* __restrict__ prm, int cstride) {
  const int img = blockIdx.y;
  const int lane = threadIdx.x & 63, q = lane & 3;
  const int an = blockIdx.x * DEC_ANCHORS + (threadIdx.x >> 2);
  const bool inside = an < a.A;
  const int ai = inside ? an : 0;
  const int idx = img * a.A + ai;
  int lv = 0;
  if (a.nlev > 1 && ai >= a.lv[1].base) lv = 1;
  if (a.nlev > 2 && ai >= a.lv[2].base) lv = 2;
  const DecodeLevel& L = a.lv[lv];
  const int local = ai - L.base;
  const int yy = local / L.W, xx = local - yy * L.W;
  const size_t pix = (size_t)img * L.H * L.W + local;

  float best = -INFINITY;
  int bcls = 0;
  const f16* cp = L.cls.p + pix * L.cls.s + L.cls.o;
  // this lane's chunks of up to 128 classes are fetched before any is consumed
  for (int c00 = 0; inside && c00 < L.cls.C; c00 += 128) {
    f16x8 v[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int c0 = c00 + 8 * (q + 4 * u);
      if (c0 < L.cls.C) v[u] = *(const f16x8*)(cp + c0);
    }
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int c0 = c00 + 8 * (q + 4 * u);
      if (c0 >= L.cls.C) break;
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const int cl = c0 + j;
        const float f = (float)v[u][j];
        if (cl < a.nc && f > best) { best = f; bcls = cl; }
      }
    }
  }
#pragma unroll
  for (int o = 1; o < 4; o <<= 1) {
    const float ob = __shfl_xor(best, o);
    const int oc = __shfl_xor(bcls, o);
    if (ob > best || (ob == best && oc < bcls)) { best = ob; bcls = oc; }
  }
  const float score = 1.f / (1.f + expf(-best));
  const bool keep = inside && score >= prm->conf;   // the same in the anchor's four lanes
  const f16* bp = L.box.p + pix * L.box.s + L.box.o + 16 * q;
  f16x8 b0, b1;
  if (keep) {
    b0 = *(const f16x8*)(bp);
    b1 = *(const f16x8*)(bp + 8);
  }
  const unsigned long long bal = __ballot(keep && q == 0);
  if (bal) {
    const int leader = __ffsll((long long)bal) - 1;
    int base = 0;
    if (lane == leader) base = atomicAdd(&count[img], __popcll(bal));
    base = __shfl(base, leader);
    const int pos = base + __popcll(bal & ((1ull << lane) - 1ull));
    if (keep && q == 0 && pos < a.A) lst[(size_t)img * a.A + pos] = packKey(score, an);
  }
  if (!keep) return;

  // side q's expectation (bins 16q .. 16q+15), then every side to every lane of the anchor
  float dq;
  {
    float l[16];
#pragma unroll
    for (int j = 0; j < 8; j++) { l[j] = (float)b0[j]; l[j + 8] = (float)b1[j]; }
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
    dq = e / sum;
  }
  const int g0 = lane & ~3;
  const float d[4] = {__shfl(dq, g0), __shfl(dq, g0 + 1), __shfl(dq, g0 + 2), __shfl(dq, g0 + 3)};
  float* o = cand + (size_t)idx * cstride;
  if (!OBB && a.nm > 0) {   // mask coefficients: lane q copies chunks q, q + 4, ...
    const f16* mp = L.coef.p + pix * L.coef.s + L.coef.o;
    for (int c0 = 8 * q; c0 < a.nm; c0 += 32) {
      const f16x8 v = *(const f16x8*)(mp + c0);
#pragma unroll
      for (int j = 0; j < 8; j++) o[6 + c0 + j] = (float)v[j];
    }
  }
  if (q != 0) return;
  const float cx = (float)xx + 0.5f, cy = (float)yy + 0.5f, st = (float)L.stride;
  if (OBB) {
    const float t0 = (float)L.coef.p[pix * L.coef.s + L.coef.o];
    const float th = (1.f / (1.f + expf(-t0)) - 0.25f) * 3.14159265358979f;
    const float xf = (d[2] - d[0]) * 0.5f, yf = (d[3] - d[1]) * 0.5f;
    const float cs = cosf(th), sn = sinf(th);
    o[0] = (cx + xf * cs - yf * sn) * st;
    o[1] = (cy + xf * sn + yf * cs) * st;
    o[2] = (d[0] + d[2]) * st;
    o[3] = (d[1] + d[3]) * st;
    o[4] = score;
    o[5] = (float)bcls;
    o[6] = th;
    return;
  }
  o[0] = (cx - d[0]) * st;
  o[1] = (cy - d[1]) * st;
  o[2] = (cx + d[2]) * st;
  o[3] = (cy + d[3]) * st;
  o[4] = score;
  o[5] = (float)bcls;
}

void launchDecode(const DecodeArgs& a, float* cand, unsigned long long* lst, int* count,
                  const PostParams* prm, int Bn, hipStream_t st) {
  const dim3 grid((a.A + DEC_ANCHORS - 1) / DEC_ANCHORS, Bn);
  if (a.obb)
    k_decode<true><<<grid, 4 * DEC_ANCHORS, 0, st>>>(a, cand, lst, count, prm, 7);
  else
    k_decode<false><<<grid, 4 * DEC_ANCHORS, 0, st>>>(a, cand, lst, count, prm, 6 + a.nm);
}

// ------------------------------------------------------------------ NMS
// One block (16 waves) per image, on the candidate list the decode kernel appended.
//  1. selection + ranking by the total order (score desc, anchor asc) packed in one u64
//     key (selectAndRank below), so the list's arrival order never matters;
//  2. greedy suppression (k_nms semantics, engine/engine.cu:1091-1109: same class only,
//     inter/union > thr with a union > 0 guard).  Suppression never crosses classes, so
//     the greedy result is the union of independent per-class greedy passes: candidates
//     are laid out class-major (rank order within a class) and a class is decided in
//     chunks of 64 members, one member per lane: each survivor in turn strikes the later
//     members of its chunk that it suppresses (greedyChunk).  A class of at most 64
//     members is one wave's work; in a larger one, a chunk's survivors then strike the
//     class's later members before the next chunk (one wave up to NMS_WAVE_CLASS members,
//     the whole block above).  This is exactly the sequential greedy result; survivors are
//     flagged by rank and a block prefix sum over the flags gives their output slots;
//  3. the list counter is re-armed (zeroed) for the next frame.
constexpr int NMS_THREADS = 1024;
constexpr int NMS_WAVE_CLASS = 256;          // largest class one wave resolves alone

// Selection + ranking shared by both NMS kernels.  Leaves the m = min(n, NMS_CAP) largest
// keys of lst[0..n) in descending order in sorted[0..m):
//  - above NMS_CAP candidates a radix select keeps the NMS_CAP largest keys (up to 8 passes
//    of 8-bit histograms from the top byte, stopping once the selected bin holds exactly
//    the keys still needed, and skipping the two anchor bytes that are constant below 2^16
//    anchors; keys are unique, so exactly NMS_CAP are >= T).  A wave's two most crowded
//    bins are added once each (wave-aggregated), the rest with plain LDS atomics;
//  - up to 512 keys: rank = number of strictly larger keys, TPK threads (adjacent lanes)
//    sharing a key's scan and adding their counts with shuffles; above that a bitonic sort
//    (descending) of the keys padded with zeros to 1024 or 2048 (log2(P)(log2(P)+1)/2
//    compare-exchange steps instead of P^2 compares).
// `skey` (NMS_CAP keys) stages the selected keys and must not alias `sorted`.  Every thread
// of the block calls it; it ends with a barrier.
struct RankShared {
  int hist[256];
  unsigned long long prefix;
  int need, count, done;
};

__device__ void selectAndRank(const unsigned long long* __restrict__ lst, int n, int A,
                              unsigned long long* skey, unsigned long long* sorted, RankShared& rs) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int m = min(n, NMS_CAP);
  if (n > NMS_CAP) {
    if (tid == 0) { rs.prefix = 0ull; rs.need = NMS_CAP; rs.count = 0; rs.done = 0; }
    for (int p = 0; p < 8; p++) {
      const int shift = 56 - 8 * p;
      if (p == 4 && A <= 65536) {
        // the low word is 0xFFFFFFFF - anchor: with fewer than 2^16 anchors its top two bytes
        // are 0xFF for every key, so those two passes would select bin 255 twice
        __syncthreads();
        if (tid == 0) rs.prefix |= 0xFFFF0000ull;
        p = 5;
        continue;
      }
      for (int i = tid; i < 256; i += NMS_THREADS) rs.hist[i] = 0;
      __syncthreads();
      const unsigned long long pre = rs.prefix;
      auto count = [&](unsigned long long k, bool valid) {
        int bin = -1;
        if (valid && (p == 0 || (k >> (shift + 8)) == (pre >> (shift + 8)))) bin = (int)((k >> shift) & 255);
        // crowded bins (the leading bytes of scores) are added once per wave for the first
        // two distinct bins; lanes left over hit spread-out bins with plain atomics
        unsigned long long todo = __ballot(bin >= 0);
#pragma unroll
        for (int peel = 0; peel < 2 && todo; peel++) {
          const int leader = __ffsll((long long)todo) - 1;
          const int lb = __shfl(bin, leader);
          const unsigned long long same = __ballot(bin == lb);
          if (lane == leader) atomicAdd(&rs.hist[lb], __popcll(same));
          if (bin == lb) bin = -1;
          todo &= ~same;
        }
        if (bin >= 0) atomicAdd(&rs.hist[bin], 1);
      };
      for (int i0 = 0; i0 < n; i0 += NMS_THREADS) {
        const int i = i0 + tid;
        count(i < n ? lst[i] : 0ull, i < n);
      }
      __syncthreads();
      // the bin holding the need-th largest key: lane l of wave 0 owns bins 255-4l .. 252-4l
      // (descending), a prefix sum over the lanes finds the one lane whose range holds it
      if (tid < 64) {
        int h[4], sum = 0;
#pragma unroll
        for (int u = 0; u < 4; u++) {
          h[u] = rs.hist[255 - 4 * lane - u];
          sum += h[u];
        }
        int incl = sum;
        for (int o = 1; o < 64; o <<= 1) {
          const int y = __shfl_up(incl, o);
          if (lane >= o) incl += y;
        }
        const int need = rs.need, excl = incl - sum;
        if (excl < need && need <= incl) {
          int cum = excl, sel = 255 - 4 * lane - 3;
#pragma unroll
          for (int u = 0; u < 4; u++) {
            if (cum + h[u] >= need) { sel = 255 - 4 * lane - u; break; }
            cum += h[u];
          }
          rs.need = need - cum;
          rs.prefix = pre | ((unsigned long long)sel << shift);
          // the bin holds exactly the keys still needed: every key with this prefix is
          // selected, so the prefix (lower bits zero) is already the threshold
          if (cum + rs.hist[sel] == need) rs.done = 1;
        }
      }
      __syncthreads();
      if (rs.done) break;   // block-uniform
    }
    const unsigned long long T = rs.prefix;
    for (int i = tid; i < n; i += NMS_THREADS) {
      const unsigned long long k = lst[i];
      if (k >= T) skey[atomicAdd(&rs.count, 1)] = k;
    }
  } else {
    for (int i = tid; i < n; i += NMS_THREADS) skey[i] = lst[i];
  }
  __syncthreads();
  static_assert(NMS_CAP == 2 * NMS_THREADS, "one compare-exchange per thread and step");
  if (m <= 512) {
    int tpk = 1;
    while (tpk < 64 && m * tpk * 2 <= NMS_THREADS) tpk *= 2;
    const int i = tid / tpk, part = tid - i * tpk;
    unsigned long long k = ~0ull;
    int r = 0;
    if (i < m) {
      k = skey[i];
      int j = part;
      for (; j + 7 * tpk < m; j += 8 * tpk) {   // 8 independent loads per trip
        unsigned long long v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = skey[j + u * tpk];
#pragma unroll
        for (int u = 0; u < 8; u++) r += v[u] > k;
      }
      for (; j < m; j += tpk) r += skey[j] > k;
    }
    for (int o = 1; o < tpk; o <<= 1) r += __shfl_xor(r, o);
    if (i < m && part == 0) sorted[r] = k;
  } else {
    const int P = m > 1024 ? 2048 : 1024;
    for (int i = m + tid; i < P; i += NMS_THREADS) skey[i] = 0ull;   // below every real key
    __syncthreads();
    for (int k = 2; k <= P; k <<= 1) {
      for (int j = k >> 1; j > 0; j >>= 1) {
        if (tid < P / 2) {
          const int i = ((tid & ~(j - 1)) << 1) | (tid & (j - 1)), l = i + j;
          const unsigned long long a = skey[i], b = skey[l];
          if ((a < b) == ((i & k) == 0)) {   // descending where (i & k) == 0
            skey[i] = b;
            skey[l] = a;
          }
        }
        __syncthreads();
      }
    }
    for (int r = tid; r < m; r += NMS_THREADS) sorted[r] = skey[r];
  }
  __syncthreads();
}

// Sequential greedy over one chunk of at most 64 members of a class, member j on lane j in
// rank order: the lowest member left in `todo` is kept, and every later member of the chunk
// that it suppresses leaves `todo` -- one ballot per survivor, the survivor's box broadcast
// by readlane, so the serial chain is the class's survivors rather than its pairs.  `todo`
// is wave-uniform and every lane of the wave calls this together; returns the kept members.
__device__ __forceinline__ unsigned long long greedyChunk(float4 bx, unsigned long long todo, float thr,
                                                          int lane) {
  unsigned long long keep = 0ull;
  while (todo) {
    const int t = __builtin_ctzll(todo);
    keep |= 1ull << t;
    const float4 bt = make_float4(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(bx.x), t)),
                                  __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bx.y), t)),
                                  __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bx.z), t)),
                                  __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bx.w), t)));
    todo &= ~(__ballot(lane > t && suppresses(bt, bx, thr)) | (1ull << t));
  }
  return keep;
}

__global__ __launch_bounds__(NMS_THREADS) void k_nms(const float* __restrict__ cand,
                                                     unsigned long long* __restrict__ lists,
                                                     int* __restrict__ counts, int A, int cstride,
                                                     float* __restrict__ out,
                                                     int* __restrict__ outidx, int* __restrict__ outcnt,
                                                     int* __restrict__ rawcnt,
                                                     const PostParams* __restrict__ prm) {
  __shared__ unsigned long long skey[NMS_CAP];
  __shared__ float4 sbox[NMS_CAP];                 // rank-ordered keys during selection, then boxes by rank
  __shared__ short scls[NMS_CAP];
  __shared__ int chist[NMS_CLASSES];
  __shared__ int cstart[NMS_CLASSES];              // class-major start of a class
  __shared__ int cfill[NMS_CLASSES];               // bucket fill counters
  __shared__ short present[NMS_CLASSES];
  __shared__ short large[NMS_CLASSES];             // classes of more than 64 members
  __shared__ short lchunk[NMS_CAP / 64][NMS_CAP / 64];   // large-class members per 64-rank chunk
  __shared__ __attribute__((aligned(16))) short bucket[NMS_CAP];   // ranks, grouped by class
  __shared__ short perm[NMS_CAP];                  // class-major position -> rank
  __shared__ float4 cbox[NMS_CAP];                 // boxes, class-major
  __shared__ unsigned removed[NMS_CAP / 32];       // kept flags by rank
  __shared__ unsigned struck[NMS_CAP / 32];        // suppressed flags, class-major (large classes)
  __shared__ float4 stepBox[64];                   // survivors of a huge class's chunk
  __shared__ int npresent, nlarge, nstep, wsum[NMS_THREADS / 64];
  __shared__ RankShared rs;
  static_assert(NMS_CLASSES == NMS_THREADS, "one class bin per thread");

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // scalar: loops over waves stay scalar
  const int img = blockIdx.x;
  const float* cimg = cand + (size_t)img * A * cstride;
  const float thr = prm->iou;
  const int maxdet = min(prm->max_det, MAX_OUT);
  const int n = min(counts[img], A);
  const int m = min(n, NMS_CAP);
  if (tid == 0) { npresent = 0; nlarge = 0; }
  chist[tid] = 0;
  cfill[tid] = 0;

  // 1. the m best keys in rank order (parked in the box array's storage); every thread
  //    lifts its entries and their candidate records into registers, counting classes
  unsigned long long* sorted = reinterpret_cast<unsigned long long*>(sbox);
  selectAndRank(lists + (size_t)img * A, n, A, skey, sorted, rs);
  for (int i = tid; i < NMS_CAP / 32; i += NMS_THREADS) removed[i] = 0u;
  for (int i = tid; i < NMS_CAP / 32; i += NMS_THREADS) struck[i] = 0u;
  unsigned long long kr[2] = {0ull, 0ull};
  float4 br[2];
  short cr[2] = {0, 0};
#pragma unroll
  for (int u = 0; u < 2; u++) {
    const int r = tid + u * NMS_THREADS;
    if (r < m) {
      kr[u] = sorted[r];
      const float* rec = cimg + (size_t)keyAnchor(kr[u]) * cstride;
      br[u] = make_float4(rec[0], rec[1], rec[2], rec[3]);
      cr[u] = (short)min(max((int)rec[5], 0), NMS_CLASSES - 1);   // ids are < nc <= NMS_CLASSES
    }
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < 2; u++) {
    const int r = tid + u * NMS_THREADS;
    if (r < m) {
      skey[r] = kr[u];
      sbox[r] = br[u];
      scls[r] = cr[u];
      atomicAdd(&chist[cr[u]], 1);
    }
  }
  __syncthreads();

  // 2. class-major layout (ranks grouped by class, rank order inside a class).  Thread t
  //    owns class t: the classes present, the large ones (> 64 members), and the exclusive
  //    prefix of the histogram.  A rank of a small class drops into its class's bucket (any
  //    order) and finds its place by counting the class members of smaller rank.  Large
  //    classes are placed by 64-rank chunks: one ballot per (chunk, large class) counts the
  //    class in the chunk, a prefix over chunks gives each chunk's start in the class, and
  //    a member's place adds its ballot prefix within the chunk.
  {
    const int h = chist[tid];
    if (h > 0) present[atomicAdd(&npresent, 1)] = (short)tid;
    if (h > 64) large[atomicAdd(&nlarge, 1)] = (short)tid;
    int incl = h;
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(incl, o);
      if (lane >= o) incl += y;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int off = 0;
    for (int w = 0; w < wave; w++) off += wsum[w];
    cstart[tid] = off + incl - h;
  }
  __syncthreads();
  const int nch = (m + 63) >> 6;           // 64-rank chunks (<= 32)
#pragma unroll
  for (int u = 0; u < 2; u++) {
    const int r = tid + u * NMS_THREADS;
    if (r < m && chist[cr[u]] <= 64) bucket[cstart[cr[u]] + atomicAdd(&cfill[cr[u]], 1)] = (short)r;
  }
  for (int q = wave; q < nch; q += NMS_THREADS / 64) {
    const int r = 64 * q + lane;
    const int c = r < m ? scls[r] : -1;
    for (int li = 0; li < nlarge; li++) {
      const int cnt = __popcll(__ballot(c == large[li]));
      if (lane == 0) lchunk[q][li] = (short)cnt;
    }
  }
  __syncthreads();
  if (tid < nlarge) {
    int run = 0;
    for (int q = 0; q < nch; q++) {
      const int v = lchunk[q][tid];
      lchunk[q][tid] = (short)run;
      run += v;
    }
  }
  __syncthreads();
  for (int q = wave; q < nch; q += NMS_THREADS / 64) {
    const int r = 64 * q + lane;
    const int c = r < m ? scls[r] : -1;
    for (int li = 0; li < nlarge; li++) {
      const unsigned long long bal = __ballot(c == large[li]);
      if (c == large[li]) {
        const int pos = cstart[c] + lchunk[q][li] + __popcll(bal & ((1ull << lane) - 1ull));
        perm[pos] = (short)r;
        cbox[pos] = sbox[r];
      }
    }
  }
#pragma unroll
  for (int u = 0; u < 2; u++) {
    const int r = tid + u * NMS_THREADS;
    if (r < m && chist[cr[u]] <= 64) {
      const int sc = cstart[cr[u]], se = sc + chist[cr[u]];
      int below = 0;
      for (int c8 = sc & ~7; c8 < se; c8 += 8) {     // 16-byte reads of the class's bucket
        const short4 lo = *reinterpret_cast<const short4*>(&bucket[c8]);
        const short4 hi = *reinterpret_cast<const short4*>(&bucket[c8 + 4]);
        const short v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
        for (int e = 0; e < 8; e++) below += (c8 + e >= sc && c8 + e < se && v[e] < r) ? 1 : 0;
      }
      perm[sc + below] = (short)r;
      cbox[sc + below] = br[u];
    }
  }
  __syncthreads();

  // 4. per-class greedy.  `removed` holds the kept flag of every candidate by rank.
  //  4a. a class of at most 64 members is one chunk, resolved by one wave (greedyChunk;
  //      waves take the classes round-robin)
  const int npres = uni(npresent), nlrg = uni(nlarge);
  for (int pc = wave; pc < npres; pc += NMS_THREADS / 64) {
    const int c = uni(present[pc]);
    const int sc = uni(cstart[c]), g = uni(chist[c]);
    if (g > 64) continue;                   // wave-uniform
    const bool valid = lane < g;
    const int mine = valid ? perm[sc + lane] : 0;
    const float4 bx = valid ? cbox[sc + lane] : make_float4(0.f, 0.f, 0.f, 0.f);
    const unsigned long long keep = greedyChunk(bx, g >= 64 ? ~0ull : ((1ull << g) - 1ull), thr, lane);
    if ((keep >> lane) & 1ull) atomicOr(&removed[mine >> 5], 1u << (mine & 31));
  }
  //  4b. a class of 65 .. NMS_WAVE_CLASS members: one wave, chunk by chunk -- the chunk is
  //      resolved by greedyChunk (members struck by earlier chunks excluded), then the lanes
  //      strike the class's later members that a survivor of the chunk suppresses
  //      (survivor boxes broadcast by readlane).  Waves take such classes round-robin; a
  //      class stops once it has max_det survivors (a later survivor ranks below max_det
  //      others and never reaches the output).
  for (int li = wave; li < nlrg; li += NMS_THREADS / 64) {
    const int c = uni(large[li]);
    const int sc = uni(cstart[c]), g = uni(chist[c]);
    if (g > NMS_WAVE_CLASS) continue;       // wave-uniform: 4c below
    int K = 0;
    for (int q0 = 0; q0 < g && K < maxdet; q0 += 64) {
      const int gq = min(64, g - q0);
      const int p = sc + q0 + lane;
      const bool valid = lane < gq;
      const int mine = valid ? perm[p] : 0;
      const float4 bx = valid ? cbox[p] : make_float4(0.f, 0.f, 0.f, 0.f);
      const bool gone = valid && ((struck[p >> 5] >> (p & 31)) & 1u);
      const unsigned long long keep =
          greedyChunk(bx, (gq >= 64 ? ~0ull : ((1ull << gq) - 1ull)) & ~__ballot(gone), thr, lane);
      if ((keep >> lane) & 1ull) atomicOr(&removed[mine >> 5], 1u << (mine & 31));
      K += __popcll(keep);
      for (int p0 = sc + q0 + 64; p0 < sc + g; p0 += 64) {
        const int pp = p0 + lane;
        bool live = pp < sc + g && !((struck[pp >> 5] >> (pp & 31)) & 1u);
        const float4 bq = live ? cbox[pp] : make_float4(0.f, 0.f, 0.f, 0.f);
        bool hit = false;
        // up to 4 survivors per round (independent tests; a member is struck when any
        // survivor of the chunk suppresses it, whatever the order)
        for (unsigned long long kk = keep; kk && __ballot(live && !hit);) {
          bool h = false;
#pragma unroll
          for (int u = 0; u < 4; u++) {
            if (kk) {
              const int t = __builtin_ctzll(kk);
              kk &= kk - 1ull;
              const float4 bi = make_float4(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(bx.x), t)),
                                            __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bx.y), t)),
                                            __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bx.z), t)),
                                            __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bx.w), t)));
              h |= suppresses(bi, bq, thr);
            }
          }
          if (live && h) hit = true;
        }
        if (hit) atomicOr(&struck[pp >> 5], 1u << (pp & 31));
      }
    }
  }
  __syncthreads();
  //  4c. a larger class goes chunk by chunk with the whole block: wave 0 resolves the chunk
  //      (greedyChunk),
  //      then every thread strikes later members of the class that a survivor of the chunk
  //      suppresses (survivor boxes read as LDS broadcasts)
  for (int li = 0; li < nlrg; li++) {
    const int c = uni(large[li]);
    const int sc = uni(cstart[c]), g = uni(chist[c]);
    if (g <= NMS_WAVE_CLASS) continue;      // block-uniform
    int K = 0;
    for (int q0 = 0; q0 < g && K < maxdet; q0 += 64) {
      const int gq = min(64, g - q0);
      if (wave == 0) {
        const int p = sc + q0 + lane;
        const bool valid = lane < gq;
        const int mine = valid ? perm[p] : 0;
        const float4 bx = valid ? cbox[p] : make_float4(0.f, 0.f, 0.f, 0.f);
        const bool gone = valid && ((struck[p >> 5] >> (p & 31)) & 1u);
        const unsigned long long keep =
            greedyChunk(bx, (gq >= 64 ? ~0ull : ((1ull << gq) - 1ull)) & ~__ballot(gone), thr, lane);
        if ((keep >> lane) & 1ull) {
          atomicOr(&removed[mine >> 5], 1u << (mine & 31));
          stepBox[__popcll(keep & ((1ull << lane) - 1ull))] = bx;
        }
        if (lane == 0) nstep = __popcll(keep);
      }
      __syncthreads();
      const int Kq = uni(nstep);
      K += Kq;
      for (int p = sc + q0 + 64 + tid; p < sc + g && Kq > 0; p += NMS_THREADS) {
        if ((struck[p >> 5] >> (p & 31)) & 1u) continue;
        const float4 bp = cbox[p];
        for (int k = 0; k < Kq; k += 4) {   // 4 survivor boxes per round, requested together
          float4 sb[4];
#pragma unroll
          for (int u = 0; u < 4; u++) sb[u] = stepBox[min(k + u, Kq - 1)];
          bool h = false;
#pragma unroll
          for (int u = 0; u < 4; u++) h |= k + u < Kq && suppresses(sb[u], bp, thr);
          if (h) {
            atomicOr(&struck[p >> 5], 1u << (p & 31));
            break;
          }
        }
      }
      __syncthreads();
    }
  }
  __syncthreads();

  // 5. output slots: exclusive prefix count of kept flags in rank order (thread t owns
  //    ranks 2t, 2t+1); records come from the candidate array
  const int r0 = 2 * tid, r1 = 2 * tid + 1;
  const int f0 = r0 < m ? (removed[r0 >> 5] >> (r0 & 31)) & 1 : 0;
  const int f1 = r1 < m ? (removed[r1 >> 5] >> (r1 & 31)) & 1 : 0;
  const int v = f0 + f1;
  int incl = v;
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o);
    if (lane >= o) incl += y;
  }
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  int off = 0;
  for (int w = 0; w < wave; w++) off += wsum[w];
  const int ex = off + incl - v;
  auto emit = [&](int i, int slot) {
    const int an = keyAnchor(skey[i]);
    const float* rec = cimg + (size_t)an * cstride;
    float* d = out + ((size_t)img * MAX_OUT + slot) * 6;
    d[0] = rec[0]; d[1] = rec[1]; d[2] = rec[2]; d[3] = rec[3];
    d[4] = __uint_as_float((unsigned)(skey[i] >> 32));
    d[5] = (float)scls[i];
    outidx[img * MAX_OUT + slot] = an;
  };
  if (f0 && ex < maxdet) emit(r0, ex);
  if (f1 && ex + f0 < maxdet) emit(r1, ex + f0);
  if (tid == NMS_THREADS - 1) {
    outcnt[img] = min(off + incl, maxdet);
    rawcnt[img] = n;
    counts[img] = 0;   // re-arm the decode list for the next frame
  }
}

// ------------------------------------------------------------------ rotated NMS (OBB)
// One block (16 waves) per image.  ultralytics fast-NMS semantics, as k_nms_obb
// (engine/engine.cu:1178-1252): candidate j is dropped iff some higher-ranked candidate
// of its class, suppressed or not, has probiou >= thr with it.  There is no sequential
// dependence, so every candidate is decided independently:
//  1. selection + ranking by (score desc, anchor asc), as for detect;
//  2. each thread owns ranks 2t, 2t+1: it loads their records and turns (w, h, theta) into
//     the covariance terms once (a = w^2/12, b = h^2/12, A = a cos^2 + b sin^2,
//     B = a sin^2 + b cos^2, C = (a - b) cos sin, engine/engine.cu:1199-1204);
//  3. the ranks are grouped by class (a class histogram, its prefix sum, then one wave per
//     class gathering the class's ranks in order with ballots), so the lanes of a wave
//     decide candidates of one class and scan the same higher-ranked members together;
//  4. lane p of a wave decides class-major position p; the wave walks the higher-ranked
//     positions of its lanes' classes together and first applies a cheap exact bound: for
//     covariances with determinant >= 1, bd >= |d|^2 / (4 trace(S1 + S2)), and iou >= thr
//     needs bd <= B* = -ln(1 + eps - (1 - thr)^2), so |d|^2 > 8 B* trace (a factor-2
//     margin) rules a pair out.  The bound is used for 0.05 <= thr <= 0.95 and for boxes
//     whose covariance condition number is below ~1e4, where fp32 rounding of the full
//     expression stays far inside that margin.  Pairs it cannot rule out go to a per-wave
//     LDS queue; each 64 queued pairs are evaluated exactly, one pair per lane, so the
//     transcendental path runs on full waves;
//  5. survivors take output slots by a block prefix count in rank order (max_det cap).
constexpr int OBB_QUEUE = 128;               // per-wave queue of pairs for exact evaluation

__global__ __launch_bounds__(NMS_THREADS) void k_nms_obb(const float* __restrict__ cand,
                                                         unsigned long long* __restrict__ lists,
                                                         int* __restrict__ counts, int A,
                                                         float* __restrict__ out,
                                                         int* __restrict__ outidx,
                                                         int* __restrict__ outcnt,
                                                         int* __restrict__ rawcnt,
                                                         const PostParams* __restrict__ prm) {
  // regionA: ranked keys during selection, then (A, B, C, class) per rank
  // regionB: staged keys during selection, then (x, y) per rank
  __shared__ float4 regionA[NMS_CAP];
  __shared__ unsigned long long regionB[NMS_CAP];
  __shared__ short perm[NMS_CAP];             // class-major position -> rank
  __shared__ int cstart[NMS_CLASSES];         // class histogram, then its exclusive prefix
  __shared__ short present[NMS_CLASSES];
  __shared__ unsigned dead[NMS_CAP / 32];
  __shared__ RankShared rs;
  __shared__ int wsum[NMS_THREADS / 64];
  __shared__ int npresent;
  __shared__ float4 ppos[NMS_CAP];            // class-major: x, y, trace (-1: no bound)
  __shared__ unsigned queue[NMS_THREADS / 64][OBB_QUEUE];
  static_assert(NMS_CLASSES == NMS_THREADS, "one class bin per thread");

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // scalar: loops over waves stay scalar
  const int img = blockIdx.x;
  const float* cimg = cand + (size_t)img * A * 7;
  const float thr = prm->iou;
  const int maxdet = min(prm->max_det, MAX_OUT);
  const int n = min(counts[img], A);
  const int m = min(n, NMS_CAP);
  const float bstar = (thr >= 0.05f && thr <= 0.95f) ? -logf(1.f + 1e-7f - (1.f - thr) * (1.f - thr)) : 0.f;
  const float skipK = bstar > 0.f ? 8.f * bstar : INFINITY;

  unsigned long long* sorted = reinterpret_cast<unsigned long long*>(regionA);
  selectAndRank(lists + (size_t)img * A, n, A, regionB, sorted, rs);
  for (int i = tid; i < NMS_CAP / 32; i += NMS_THREADS) dead[i] = 0u;
  cstart[tid] = 0;
  if (tid == 0) npresent = 0;
  unsigned long long kr[2] = {0ull, 0ull};
  float4 gr[2];
  float2 pr[2];
#pragma unroll
  for (int u = 0; u < 2; u++) {
    const int r = 2 * tid + u;
    if (r < m) {
      kr[u] = sorted[r];
      const float* rec = cimg + (size_t)keyAnchor(kr[u]) * 7;
      const float w = rec[2], h = rec[3], th = rec[6];
      const float a = w * w * (1.f / 12.f), b = h * h * (1.f / 12.f);
      const float cs = cosf(th), sn = sinf(th);
      const float Aa = a * cs * cs + b * sn * sn;
      const float Bb = a * sn * sn + b * cs * cs;
      const float Cc = (a - b) * cs * sn;
      const float cl = fminf(fmaxf(rec[5], 0.f), (float)(NMS_CLASSES - 1));
      gr[u] = make_float4(Aa, Bb, Cc, cl);
      pr[u] = make_float2(rec[0], rec[1]);
    }
  }
  __syncthreads();
  float2* sxy = reinterpret_cast<float2*>(regionB);
#pragma unroll
  for (int u = 0; u < 2; u++) {
    const int r = 2 * tid + u;
    if (r < m) {
      regionA[r] = gr[u];
      sxy[r] = pr[u];
      atomicAdd(&cstart[(int)gr[u].w], 1);
    }
  }
  __syncthreads();
  // 3a. classes present and the exclusive prefix of the histogram (thread t owns class t)
  {
    const int h = cstart[tid];
    if (h > 0) present[atomicAdd(&npresent, 1)] = (short)tid;
    int incl = h;
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(incl, o);
      if (lane >= o) incl += y;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int off = 0;
    for (int w = 0; w < wave; w++) off += wsum[w];
    cstart[tid] = off + incl - h;
  }
  __syncthreads();
  // 3b. one wave per class: its ranks in order, appended with ballots (no atomics)
  for (int pc = wave; pc < npresent; pc += NMS_THREADS / 64) {
    const int c = present[pc];
    const float cf = (float)c;
    int g = cstart[c];
    for (int i0 = 0; i0 < m; i0 += 64) {
      const int r = i0 + lane;
      const bool in = r < m && regionA[r].w == cf;
      const unsigned long long bal = __ballot(in);
      if (in) perm[g + __popcll(bal & ((1ull << lane) - 1ull))] = (short)r;
      g += __popcll(bal);
    }
  }
  __syncthreads();

  // class-major copies of what the cheap bound reads
  for (int p = tid; p < m; p += NMS_THREADS) {
    const int r = perm[p];
    const float4 g = regionA[r];
    const float2 xy = sxy[r];
    const float tr = g.x + g.y;
    const float det = fmaxf(g.x * g.y - g.z * g.z, 0.f);
    const bool bounded = det >= OBB_DET_MIN && det >= OBB_COND * tr * tr;
    ppos[p] = make_float4(xy.x, xy.y, bounded ? tr : -1.f, 0.f);
  }
  __syncthreads();

  // 4. fast-NMS decisions
  unsigned* wq = queue[wave];
  int qhead = 0, qtail = 0;                   // wave-uniform queue cursors
  auto flush = [&](int cnt) {                 // exact probiou of the cnt (<= 64) oldest pairs
    if (lane < cnt) {
      const unsigned e = wq[(qhead + lane) & (OBB_QUEUE - 1)];
      const int i = perm[e >> 16], j = perm[e & 0xFFFFu];
      const float4 gi = regionA[i], gj = regionA[j];
      const float di = fmaxf(gi.x * gi.y - gi.z * gi.z, 0.f);
      const float dj = fmaxf(gj.x * gj.y - gj.z * gj.z, 0.f);
      if (probiou(sxy[i], gi, di, sxy[j], gj, dj) >= thr) atomicOr(&dead[j >> 5], 1u << (j & 31));
    }
    qhead += cnt;
  };
  for (int base = wave * 64; base < m; base += NMS_THREADS) {
    const int p = base + lane;
    const bool valid = p < m;
    const int j = valid ? perm[p] : 0;
    const float4 me = valid ? ppos[p] : make_float4(0.f, 0.f, -1.f, 0.f);
    const int s = valid ? cstart[(int)regionA[j].w] : 0x7fffffff;
    bool alive = valid && s < p;              // has a higher-ranked member of its class
    int lo = s, hi = valid ? p : 0;
    for (int o = 32; o > 0; o >>= 1) {
      lo = min(lo, __shfl_xor(lo, o));
      hi = max(hi, __shfl_xor(hi, o));
    }
    float4 nxt = lo < hi ? ppos[lo] : make_float4(0.f, 0.f, -1.f, 0.f);
    for (int q = lo; q < hi; q++) {
      if (!__ballot(alive)) break;
      const float4 oi = nxt;
      if (q + 1 < hi) nxt = ppos[q + 1];      // next position's load overlaps this one's work
      const float dx = oi.x - me.x, dy = oi.y - me.y;
      const bool far = me.z > 0.f && oi.z > 0.f && dx * dx + dy * dy > skipK * (oi.z + me.z);
      const bool need = alive && q >= s && !far;
      const unsigned long long bal = __ballot(need);
      if (bal) {
        if (need) wq[(qtail + __popcll(bal & ((1ull << lane) - 1ull))) & (OBB_QUEUE - 1)] = ((unsigned)q << 16) | (unsigned)p;
        qtail += __popcll(bal);
        if (qtail - qhead >= 64) {
          flush(64);
          if (alive) alive = !((dead[j >> 5] >> (j & 31)) & 1u);
        }
      }
      alive = alive && q + 1 < p;
    }
  }
  flush(qtail - qhead);
  __syncthreads();

  // 5. output slots: exclusive prefix count of survivors in rank order (thread t owns
  //    ranks 2t, 2t+1, whose keys it still holds)
  const int r0 = 2 * tid, r1 = 2 * tid + 1;
  const int f0 = r0 < m ? !((dead[r0 >> 5] >> (r0 & 31)) & 1u) : 0;
  const int f1 = r1 < m ? !((dead[r1 >> 5] >> (r1 & 31)) & 1u) : 0;
  const int v = f0 + f1;
  int incl = v;
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o);
    if (lane >= o) incl += y;
  }
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  int off = 0;
  for (int w = 0; w < wave; w++) off += wsum[w];
  const int ex = off + incl - v;
  auto emit = [&](unsigned long long key, int slot) {
    const int an = keyAnchor(key);
    const float* rec = cimg + (size_t)an * 7;
    float* d = out + ((size_t)img * MAX_OUT + slot) * 7;
#pragma unroll
    for (int q = 0; q < 7; q++) d[q] = rec[q];
    outidx[img * MAX_OUT + slot] = an;
  };
  if (f0 && ex < maxdet) emit(kr[0], ex);
  if (f1 && ex + f0 < maxdet) emit(kr[1], ex + f0);
  if (tid == NMS_THREADS - 1) {
    outcnt[img] = min(off + incl, maxdet);
    rawcnt[img] = n;
    counts[img] = 0;   // re-arm the decode list for the next frame
  }
}

void launchNmsObb(const float* cand, unsigned long long* lists, int* counts, int A, float* out,
                  int* outidx, int* outcnt, int* rawcnt, const PostParams* prm, int Bn,
                  hipStream_t st) {
  k_nms_obb<<<Bn, NMS_THREADS, 0, st>>>(cand, lists, counts, A, out, outidx, outcnt, rawcnt, prm);
}

size_t nmsScratchBytes(int A) { return (size_t)A * sizeof(unsigned long long); }

void launchNms(const float* cand, unsigned long long* lists, int* counts, int A, int cstride,
               float* out, int* outidx, int* outcnt, int* rawcnt, const PostParams* prm, int Bn,
               hipStream_t st) {
  k_nms<<<Bn, NMS_THREADS, 0, st>>>(cand, lists, counts, A, cstride, out, outidx, outcnt, rawcnt, prm);
}

// ------------------------------------------------------------------ masks
// Survivor masks at proto resolution (k_mask_assemble, engine/engine.cu:1125-1158):
// logit = coef . proto (fp32, channels summed in order), pixel kept iff inside the box scaled
// to proto resolution (half-open float compares) and logit > 0.
// Grid (pixel tiles of 1024, groups of MSK_GROUP survivor slots, images): each thread keeps
// the proto vectors of 4 consecutive pixels in registers and walks the group's survivors
// (coefficients and boxes staged in LDS, read as broadcasts), writing 4 mask bytes per
// survivor in one store.  The proto is read once per survivor group instead of once per
// survivor.  Groups past the image's count exit, so the fixed grid can live in a graph.
constexpr int MSK_GROUP = 32;
constexpr int MSK_PIX = 4;

template <int NMC>   // 8-channel chunks of the proto (nm / 8)
__global__ __launch_bounds__(256) void k_masks(View proto, const float* __restrict__ cand, int cstride,
                                               int A, const int* __restrict__ outidx,
                                               const int* __restrict__ outcnt,
                                               const float* __restrict__ outdets,
                                               uint8_t* __restrict__ masks, float rx, float ry) {
  constexpr int NM = 8 * NMC;
  const int img = blockIdx.z, d0 = blockIdx.y * MSK_GROUP;
  const int cnt = outcnt[img];
  if (d0 >= cnt) return;   // block-uniform
  const int nd = min(MSK_GROUP, cnt - d0);
  __shared__ float co[MSK_GROUP][NM];
  __shared__ float4 bb[MSK_GROUP];
  const int t = threadIdx.x;
  for (int i = t; i < nd * NM; i += 256) {
    const int sv = i / NM, c = i - sv * NM;
    const int an = outidx[img * MAX_OUT + d0 + sv];
    co[sv][c] = cand[((size_t)img * A + an) * cstride + 6 + c];
  }
  if (t < nd) {
    const float* det = outdets + ((size_t)img * MAX_OUT + d0 + t) * 6;
    bb[t] = make_float4(det[0] * rx, det[1] * ry, det[2] * rx, det[3] * ry);
  }
  const int Ph = proto.H, Pw = proto.W, HW = Ph * Pw;
  const int p0 = (blockIdx.x * 256 + t) * MSK_PIX;
  const f16* pimg = proto.p + (size_t)img * HW * proto.s + proto.o;
  f16x8 pv[MSK_PIX][NMC];
  float fx[MSK_PIX], fy[MSK_PIX];
#pragma unroll
  for (int u = 0; u < MSK_PIX; u++) {
    const int p = min(p0 + u, HW - 1);
#pragma unroll
    for (int k = 0; k < NMC; k++) pv[u][k] = *(const f16x8*)(pimg + (size_t)p * proto.s + 8 * k);
    fx[u] = (float)(p % Pw);
    fy[u] = (float)(p / Pw);
  }
  __syncthreads();
  if (p0 >= HW) return;
  const bool whole = p0 + MSK_PIX <= HW && HW % MSK_PIX == 0;
  for (int sv = 0; sv < nd; sv++) {
    const float4 b = bb[sv];
    unsigned word = 0u;
#pragma unroll
    for (int u = 0; u < MSK_PIX; u++) {
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < NMC; k++)
#pragma unroll
        for (int j = 0; j < 8; j++) acc = acc + co[sv][8 * k + j] * (float)pv[u][k][j];
      const bool in = fx[u] >= b.x && fx[u] < b.z && fy[u] >= b.y && fy[u] < b.w;
      word |= (in && acc > 0.f ? 1u : 0u) << (8 * u);
    }
    uint8_t* mo = masks + ((size_t)img * MAX_OUT + d0 + sv) * HW + p0;
    if (whole) {
      *(unsigned*)mo = word;
    } else {
      for (int u = 0; u < MSK_PIX && p0 + u < HW; u++) mo[u] = (uint8_t)(word >> (8 * u));
    }
  }
}

// MFMA form (nm a multiple of 32, proto planes of whole 64-pixel tiles).  A 16-pixel x
// 16-survivor tile of logits is one v_mfma_f32_16x16x32_f16 per 32 channels with the pixels as
// the rows, so lane l ends up with 4 consecutive pixels (rows 4(l/16) .. +3) of survivor l % 16
// and writes their 4 mask bytes in one store.  The fp32 coefficients enter as fp16 hi + lo parts
// (two MFMAs; hi + lo keeps 22 of their 24 significand bits), the proto is fp16 already, and the
// products accumulate in fp32: the logits differ from an fp32 dot product in their last bits
// only, so only a logit within rounding of 0 can take the other mask bit.
// Grid (64-pixel tiles, groups of MSKM_SV survivor slots, images): wave w takes pixels
// 16w .. 16w + 15 of the tile against the group's 16-survivor tiles.  Groups past the image's
// count exit, as in k_masks.  (256-pixel tiles, staging a group's coefficients once for four
// times the pixels, measured no faster.)
constexpr int MSKM_SV = 64;
typedef float f32x4m __attribute__((ext_vector_type(4)));

template <int NMK>   // 32-channel steps of the proto (nm / 32)
__global__ __launch_bounds__(256) void k_masks_mfma(View proto, const float* __restrict__ cand, int cstride,
                                                    int A, const int* __restrict__ outidx,
                                                    const int* __restrict__ outcnt,
                                                    const float* __restrict__ outdets,
                                                    uint8_t* __restrict__ masks, float rx, float ry) {
  constexpr int NM = 32 * NMK, CP = NM + 8;   // coefficient row pitch (halves)
  const int img = blockIdx.z, d0 = blockIdx.y * MSKM_SV;
  const int cnt = outcnt[img];
  if (d0 >= cnt) return;   // block-uniform
  const int nd = min(MSKM_SV, cnt - d0);
  __shared__ __attribute__((aligned(16))) f16 chi[MSKM_SV * CP];
  __shared__ __attribute__((aligned(16))) f16 clo[MSKM_SV * CP];
  __shared__ float4 bb[MSKM_SV];
  const int t = threadIdx.x;
  for (int i = t; i < MSKM_SV * NM; i += 256) {
    const int sv = i / NM, c = i - sv * NM;
    float v = 0.f;
    if (sv < nd) {
      const int an = outidx[img * MAX_OUT + d0 + sv];
      v = cand[((size_t)img * A + an) * cstride + 6 + c];
    }
    const f16 h = (f16)v;
    chi[sv * CP + c] = h;
    clo[sv * CP + c] = (f16)(v - (float)h);
  }
  if (t < MSKM_SV) {
    float4 b = make_float4(0.f, 0.f, 0.f, 0.f);   // slots past the count: an empty box
    if (t < nd) {
      const float* det = outdets + ((size_t)img * MAX_OUT + d0 + t) * 6;
      b = make_float4(det[0] * rx, det[1] * ry, det[2] * rx, det[3] * ry);
    }
    bb[t] = b;
  }
  const int lane = t & 63, wave = t >> 6, lr = lane & 15, lg = lane >> 4;
  const int Pw = proto.W, HW = proto.H * Pw;
  const int pt = blockIdx.x * 64 + wave * 16;   // the wave's 16 pixels
  const f16* pimg = proto.p + (size_t)img * HW * proto.s + proto.o;
  f16x8 a[NMK];
#pragma unroll
  for (int s = 0; s < NMK; s++) a[s] = *(const f16x8*)(pimg + (size_t)(pt + lr) * proto.s + 32 * s + 8 * lg);
  const int q0 = pt + 4 * lg;                   // the lane's 4 output pixels
  float fx[4], fy[4];
#pragma unroll
  for (int e = 0; e < 4; e++) {
    fx[e] = (float)((q0 + e) % Pw);
    fy[e] = (float)((q0 + e) / Pw);
  }
  __syncthreads();
  for (int st = 0; 16 * st < nd; st++) {        // wave-uniform
    const int sv = 16 * st + lr;
    f32x4m acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < NMK; s++) {
      const f16x8 bh = *(const f16x8*)&chi[sv * CP + 32 * s + 8 * lg];
      const f16x8 bl = *(const f16x8*)&clo[sv * CP + 32 * s + 8 * lg];
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[s], bh, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[s], bl, acc, 0, 0, 0);
    }
    const float4 b = bb[sv];
    unsigned word = 0u;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const bool in = fx[e] >= b.x && fx[e] < b.z && fy[e] >= b.y && fy[e] < b.w;
      word |= (in && acc[e] > 0.f ? 1u : 0u) << (8 * e);
    }
    if (sv < nd) *(unsigned*)(masks + ((size_t)img * MAX_OUT + d0 + sv) * HW + q0) = word;
  }
}

void launchMasks(const View& proto, const float* cand, int cstride, int A, int nm,
                 const int* outidx, const int* outcnt, const float* outdets, uint8_t* masks,
                 float rx, float ry, int Bn, hipStream_t st) {
  const int HW = proto.H * proto.W;
  if (nm % 32 == 0 && nm <= 64 && HW % 64 == 0) {
    const dim3 g((unsigned)(HW / 64), (MAX_OUT + MSKM_SV - 1) / MSKM_SV, Bn);
    if (nm == 32)
      k_masks_mfma<1><<<g, 256, 0, st>>>(proto, cand, cstride, A, outidx, outcnt, outdets, masks, rx, ry);
    else
      k_masks_mfma<2><<<g, 256, 0, st>>>(proto, cand, cstride, A, outidx, outcnt, outdets, masks, rx, ry);
    return;
  }
  dim3 grid((HW + 256 * MSK_PIX - 1) / (256 * MSK_PIX), (MAX_OUT + MSK_GROUP - 1) / MSK_GROUP, Bn);
  switch (nm / 8) {
#define MSK(n) case n: k_masks<n><<<grid, 256, 0, st>>>(proto, cand, cstride, A, outidx, outcnt, outdets, masks, rx, ry); break;
    MSK(1) MSK(2) MSK(3) MSK(4) MSK(5) MSK(6) MSK(7) MSK(8)
#undef MSK
    default: break;
  }
}

}  // namespace yolo
