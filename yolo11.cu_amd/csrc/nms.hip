// Greedy same-class NMS for detect / segment frames, spread over many CUs.
//
// Semantics are those of k_nms (engine/engine.cu:1048-1123): the NMS_CAP best candidates by
// (score desc, anchor asc) enter; a candidate survives iff no surviving higher-ranked
// candidate of its class has inter/union > thr with it; survivors are emitted in rank order
// up to max_det.  Suppression never crosses classes, so the greedy result is the union of
// independent per-class greedy passes, and a pass only needs, for each member, which later
// members of its class it suppresses.  Six launches, each over all images of the batch:
//   1. k_nms_select  (one block per image)  a threshold key T such that the keys >= T are a
//      superset of the NMS_CAP best with at most NMS_SEL members (histogram passes over
//      the key range, each narrowing the boundary bin by 11 bits), then a gather of those
//      keys with their boxes and classes;
//   2. k_nms_rank    (many waves per image) rank = number of larger selected keys, and the
//      rank within the class = number of larger keys of the same class: every (64 keys x
//      256 keys) tile is one wave's item, partial counts meet in one packed atomic add;
//   3. k_nms_layout  (one block per image)  class histogram of the NMS_CAP best, class
//      starts, the class-major order (class start + rank within the class), the list of
//      present classes and the suppression tiles of each class;
//   4. k_nms_masks   (many waves per image) one wave per (row chunk, column chunk) tile of a
//      class: lane i tests its member against the 64 members of the column chunk;
//   5. k_nms_greedy  (one wave per class)   column by column: the members of chunk d that
//      earlier survivors suppress (an OR over their mask words), then a bit scan of the
//      chunk with its own words; stops at max_det survivors in the class;
//   6. k_nms_emit    (one block per image)  survivor flags by rank, a prefix count, records.
// Every launch leaves the workspace ready for the next frame (rank accumulators zeroed by
// the gather, survivor flags and the decode list counter by the emit).
#include "boxes.hpp"

namespace yolo {

constexpr int BLK = 1024;                 // threads of the per-image blocks
constexpr int SEL_BINS = 2048;            // 11-bit digits
constexpr int SEL_KPT = 8;                // keys a select thread keeps in registers
constexpr int RANK_TILES = NMS_SEL / 64;  // 64-key tiles of a full selection
constexpr int RANK_PART = NMS_SEL / NMS_RANK_SPLIT;
constexpr int MASK_BLOCKS = 256;          // per image; a block takes one tile at a time
constexpr int GREEDY_BLOCKS = 64;         // 4-wave blocks per image
constexpr int GREEDY_LDS_WORDS = 8192;    // a class mask up to 64 KB is resolved from LDS
static_assert(SEL_BINS == 2 * BLK && NMS_CAP == 2 * BLK && NMS_CLASSES == BLK, "one thread per two bins / ranks, one per class");
static_assert(NMS_SEL % 64 == 0 && NMS_SEL % NMS_RANK_SPLIT == 0 && RANK_PART <= BLK, "rank tiling");

// Inclusive scan of one int per thread over an NT-thread block; `total` gets the block sum.
// Every thread calls it; it ends with a barrier, so `wsum` can be reused at once.
template <int NT>
__device__ int blockScan(int v, int* wsum, int& total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o);
    if (lane >= o) incl += y;
  }
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  int off = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < NT / 64; w++) {
    const int s = wsum[w];
    off += w < wave ? s : 0;
    tot += s;
  }
  total = tot;
  __syncthreads();
  return off + incl;
}

// The same for one 64-bit value per thread (sums must not overflow their packed fields).
template <int NT>
__device__ unsigned long long blockScan64(unsigned long long v, unsigned long long* wsum,
                                          unsigned long long& total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  unsigned long long incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const unsigned long long y = __shfl_up(incl, o);
    if (lane >= o) incl += y;
  }
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  unsigned long long off = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < NT / 64; w++) {
    const unsigned long long s = wsum[w];
    off += w < wave ? s : 0;
    tot += s;
  }
  total = tot;
  __syncthreads();
  return off + incl;
}

__device__ __forceinline__ unsigned long long readlane64(unsigned long long v, int l) {
  const unsigned lo = __builtin_amdgcn_readlane((unsigned)v, l);
  const unsigned hi = __builtin_amdgcn_readlane((unsigned)(v >> 32), l);
  return ((unsigned long long)hi << 32) | lo;
}

// suppresses() with both areas computed beforehand (the same expressions, so the same fp32
// values) and the rare near-tie division taken as a wave-uniform branch.  Every lane of the
// wave must call it together.
__device__ __forceinline__ bool suppressesWave(float4 a, float aarea, float4 b, float barea, float thr) {
  const float xx1 = fmx(a.x, b.x), yy1 = fmx(a.y, b.y);
  const float xx2 = fmn(a.z, b.z), yy2 = fmn(a.w, b.w);
  const float w = fmx(0.f, xx2 - xx1), h = fmx(0.f, yy2 - yy1);
  const float inter = w * h;
  const float ua = aarea + barea - inter;
  const float p = thr * ua;
  bool s = ua > 0.f && inter > p * 1.000001f;
  const bool tie = ua > 0.f && !s && !(inter < p * 0.999999f);
  if (__ballot(tie)) {
    if (tie) s = inter / ua > thr;
  }
  return s;
}

__device__ __forceinline__ float boxArea(float4 b) { return (b.z - b.x) * (b.w - b.y); }

// ------------------------------------------------------------------ 1. select
// Every key lies in [lo, lo + 2^wbits) with lo = the conf threshold's score bits (a
// candidate has score >= conf) and the top at score 1.0.  A pass bins the keys of the
// current interval by their top 11 bits, finds the bin holding the NMS_CAP-th largest key,
// and stops if that bin and everything above it fit NMS_SEL (then T is the bin's low edge);
// otherwise the bin becomes the interval.  Keys are unique, so a 1-key-wide bin always
// fits: at most 6 passes.  Each thread keeps its first SEL_KPT keys in registers, so the
// list is read from memory once; the gather places every kept key first and then has all
// their candidate records in flight together.
template <bool OBB>
__global__ __launch_bounds__(BLK) void k_nms_select(const float* __restrict__ cand,
                                                    const unsigned long long* __restrict__ lists,
                                                    const int* __restrict__ counts, int A, int cstride,
                                                    const PostParams* __restrict__ prm,
                                                    NmsImage* __restrict__ ws) {
  __shared__ int hist[SEL_BINS];
  __shared__ int wsum[BLK / 64];
  __shared__ unsigned long long sLo;
  __shared__ int sAbove, sCnt, sCount;
  const int tid = threadIdx.x, lane = tid & 63;
  const int img = blockIdx.x;
  NmsImage& w = ws[img];
  const unsigned long long* lst = lists + (size_t)img * A;
  const int n = min(counts[img], A);
  unsigned long long kc[SEL_KPT];
#pragma unroll
  for (int u = 0; u < SEL_KPT; u++) {
    const int i = tid + u * BLK;
    kc[u] = i < n ? lst[i] : 0ull;
  }
  unsigned long long T = 0ull;
  if (n > NMS_CAP) {
    const float conf = prm->conf;
    unsigned long long lo = conf > 0.f ? (unsigned long long)__float_as_uint(conf) << 32 : 0ull;
    const unsigned long long top = (0x3F800000ull << 32) | 0xFFFFFFFFull;
    int wbits = 64 - __clzll((long long)(top - lo));
    int above = 0;
    for (int pass = 0; pass < 8; pass++) {
      const int sh = wbits > 11 ? wbits - 11 : 0;
      hist[tid] = 0;
      hist[tid + BLK] = 0;
      __syncthreads();
      auto count = [&](unsigned long long k, bool valid) {
        int bin = -1;
        const unsigned long long d = k - lo;
        if (valid && k >= lo && (d >> wbits) == 0ull) bin = (int)(d >> sh);
        // scores crowd a few bins: the wave's two most common bins take one add each
        unsigned long long todo = __ballot(bin >= 0);
#pragma unroll
        for (int peel = 0; peel < 2 && todo; peel++) {
          const int leader = __ffsll((long long)todo) - 1;
          const int lb = __shfl(bin, leader);
          const unsigned long long same = __ballot(bin == lb);
          if (lane == leader) atomicAdd(&hist[lb], __popcll(same));
          if (bin == lb) bin = -1;
          todo &= ~same;
        }
        if (bin >= 0) atomicAdd(&hist[bin], 1);
      };
#pragma unroll
      for (int u = 0; u < SEL_KPT; u++)
        if (u * BLK < n) count(kc[u], tid + u * BLK < n);
      for (int i0 = SEL_KPT * BLK; i0 < n; i0 += BLK) count(i0 + tid < n ? lst[i0 + tid] : 0ull, i0 + tid < n);
      __syncthreads();
      // thread t owns bins 2047-2t and 2046-2t: the suffix sums from the top bin down
      const int h0 = hist[SEL_BINS - 1 - 2 * tid], h1 = hist[SEL_BINS - 2 - 2 * tid];
      int total;
      const int incl = blockScan<BLK>(h0 + h1, wsum, total);
      const int excl = incl - h0 - h1;
      const int need = NMS_CAP - above;
      if (excl < need && need <= incl) {
        const bool first = excl + h0 >= need;
        const int b = first ? SEL_BINS - 1 - 2 * tid : SEL_BINS - 2 - 2 * tid;
        sLo = lo + ((unsigned long long)b << sh);
        sAbove = above + (first ? excl : excl + h0);
        sCnt = first ? h0 : h1;
      }
      __syncthreads();
      lo = sLo;
      if (sAbove + sCnt <= NMS_SEL || sh == 0) break;   // block-uniform
      above = sAbove;
      wbits = sh;
    }
    T = lo;
  }
  if (tid == 0) sCount = 0;
  __syncthreads();
  auto place = [&](unsigned long long k, bool valid) {
    const bool take = valid && k >= T;
    const unsigned long long bal = __ballot(take);
    int base = 0;
    if (lane == 0 && bal) base = atomicAdd(&sCount, __popcll(bal));
    base = __shfl(base, 0);
    const int pos = base + __popcll(bal & ((1ull << lane) - 1ull));
    return take && pos < NMS_SEL ? pos : -1;
  };
  // the record fields a candidate needs: detect x1 y1 x2 y2 . cls (6 + nm floats, 8-byte
  // aligned); rotated cx cy w h . cls theta (7 floats)
  struct Rec { float v[7]; };
  auto fetch = [&](unsigned long long k) {
    const float* rec = cand + ((size_t)img * A + keyAnchor(k)) * cstride;
    Rec r;
    if constexpr (OBB) {
#pragma unroll
      for (int q = 0; q < 7; q++) r.v[q] = rec[q];
    } else {
      const float2* r2 = (const float2*)rec;
#pragma unroll
      for (int q = 0; q < 3; q++) {
        const float2 t = r2[q];
        r.v[2 * q] = t.x;
        r.v[2 * q + 1] = t.y;
      }
      r.v[6] = 0.f;
    }
    return r;
  };
  auto store = [&](int pos, unsigned long long k, const Rec& r) {
    w.selKey[pos] = k;
    if constexpr (OBB) {
      // covariance of the rotated box, as the one-block kernel forms it (engine/engine.cu:1199-1204)
      const float a = r.v[2] * r.v[2] * (1.f / 12.f), b = r.v[3] * r.v[3] * (1.f / 12.f);
      const float cs = cosf(r.v[6]), sn = sinf(r.v[6]);
      const float Aa = a * cs * cs + b * sn * sn;
      const float Bb = a * sn * sn + b * cs * cs;
      const float Cc = (a - b) * cs * sn;
      const float tr = Aa + Bb, det = fmaxf(Aa * Bb - Cc * Cc, 0.f);
      const bool bounded = det >= OBB_DET_MIN && det >= OBB_COND * tr * tr;
      w.selBox[pos] = make_float4(r.v[0], r.v[1], bounded ? tr : -1.f, det);
      w.selAux[pos] = make_float4(Aa, Bb, Cc, 0.f);
      w.selCls[pos] = (int)fminf(fmaxf(r.v[5], 0.f), (float)(NMS_CLASSES - 1));
    } else {
      w.selBox[pos] = make_float4(r.v[0], r.v[1], r.v[2], r.v[3]);
      w.selCls[pos] = min(max((int)r.v[5], 0), NMS_CLASSES - 1);
    }
  };
  int pos[SEL_KPT];
#pragma unroll
  for (int u = 0; u < SEL_KPT; u++) pos[u] = u * BLK < n ? place(kc[u], tid + u * BLK < n) : -1;
  Rec r[SEL_KPT];
#pragma unroll
  for (int u = 0; u < SEL_KPT; u++)
    if (pos[u] >= 0) r[u] = fetch(kc[u]);
#pragma unroll
  for (int u = 0; u < SEL_KPT; u++)
    if (pos[u] >= 0) store(pos[u], kc[u], r[u]);
  for (int i0 = SEL_KPT * BLK; i0 < n; i0 += BLK) {
    const unsigned long long k = i0 + tid < n ? lst[i0 + tid] : 0ull;
    const int p = place(k, i0 + tid < n);
    if (p >= 0) store(p, k, fetch(k));
  }
  __syncthreads();
  if (tid == 0) w.selN = min(sCount, NMS_SEL);
}

// ------------------------------------------------------------------ 3. layout
// (one block per image)
// Class c with g members occupies class-major positions [start, start + g) in rank order;
// its q = ceil(g/64) chunks give q(q+1)/2 tiles (row chunk a <= column chunk b) and
// 32 q (q-1) + g mask words.  Thread t owns class t; each thread's selected keys are read
// with all their loads in flight together.
struct LayoutShared {
  int chist[NMS_CLASSES];
  int cstart[NMS_CLASSES];
  int tstart[NMS_CLASSES + 1];
  int4 info[NMS_CLASSES];       // by present-class index
  unsigned long long wsum64[BLK / 64];
};

__device__ __forceinline__ void nmsLayout(NmsImage& w, int m, bool aux, LayoutShared& L) {
  static_assert(NMS_SEL <= 3 * BLK, "three selected keys per thread");
  const int tid = threadIdx.x;
  L.chist[tid] = 0;
  const int sN = w.selN;
  // the thread's selected keys tid, tid + BLK, tid + 2 BLK: summed part ranks, class, box
  // (unconditional loads with the index clamped, so all are in flight at once)
  struct Entry { unsigned v; int c; float4 b; };
  auto load = [&](int u) {
    const int i = min(tid + u * BLK, NMS_SEL - 1);
    Entry e;
    e.v = 0u;
#pragma unroll
    for (int p = 0; p < NMS_RANK_SPLIT; p++) e.v += w.selRank[p][i];
    e.c = w.selCls[i];
    e.b = w.selBox[i];
    return e;
  };
  const Entry e0 = load(0), e1 = load(1), e2 = load(2);
  auto count = [&](const Entry& e, int u) {
    const int i = tid + u * BLK;
    if (i < sN && (int)(e.v >> 16) < m) {
      w.rIdx[e.v >> 16] = i;
      atomicAdd(&L.chist[e.c], 1);
    }
  };
  __syncthreads();
  count(e0, 0);
  count(e1, 1);
  count(e2, 2);
  __syncthreads();
  const int g = L.chist[tid];
  const int q = (g + 63) >> 6;
  const int tiles = q * (q + 1) / 2, words = g > 0 ? 32 * q * (q - 1) + g : 0;
  // one scan of the four prefixes packed in 64 bits: members (12 bits, <= 2048), present
  // classes (11 bits, <= 1024), tiles (12 bits, <= 2048) and mask words (17 bits, <= 65536)
  const unsigned long long pk = (unsigned long long)g | ((unsigned long long)(g > 0) << 12) |
                                ((unsigned long long)tiles << 23) | ((unsigned long long)words << 35);
  unsigned long long tot;
  const unsigned long long ex = blockScan64<BLK>(pk, L.wsum64, tot) - pk;
  const int gs = (int)(ex & 0xFFF), k = (int)((ex >> 12) & 0x7FF), ts = (int)((ex >> 23) & 0xFFF),
            ms = (int)(ex >> 35);
  const int P = (int)((tot >> 12) & 0x7FF), nT = (int)((tot >> 23) & 0xFFF);
  L.cstart[tid] = gs;
  if (g > 0) {
    const int4 ci = make_int4(gs, g, ms, ts);
    w.cls[k] = ci;
    L.info[k] = ci;
    L.tstart[k] = ts;
  }
  if (tid == 0) {
    L.tstart[P] = nT;
    w.nClasses = P;
    w.nTiles = nT;
  }
  __syncthreads();
  auto place = [&](const Entry& e, int u) {
    const int i = tid + u * BLK;
    const int r = (int)(e.v >> 16);
    if (i < sN && r < m) {
      const int pos = L.cstart[e.c] + (int)(e.v & 0xFFFFu);
      w.cRank[pos] = r;
      w.cBox[pos] = e.b;
      if (aux) w.cAux[pos] = w.selAux[i];
    }
  };
  place(e0, 0);
  place(e1, 1);
  place(e2, 2);
  // tile t: its class by binary search over the tile starts, then (a, b) from the local
  // index b (b + 1) / 2 + a
  for (int t = tid; t < nT; t += BLK) {
    int lo = 0, hi = P - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (L.tstart[mid] <= t) lo = mid; else hi = mid - 1;
    }
    int l = t - L.tstart[lo], b = 0;
    while (l > b) { l -= b + 1; b++; }
    const int4 ci = L.info[lo];
    w.tile[t] = make_int4(ci.x, ci.y, ci.z, (l << 5) | b);
  }
}

// ------------------------------------------------------------------ 2. rank
// Block (tile, part): lane i of every wave holds selected key tile*64+i; part p of the
// selection is staged in LDS and split over the 16 waves, each counting the larger keys of
// its share (and those of the key's class) from LDS broadcasts; the wave counts are summed
// in LDS and stored as the part's (rank << 16 | class rank).  The last block to finish an
// image (a counter) sums the parts and lays the image out.
// Block (tile, part): lane i of every wave holds selected key tile*64+i; part p of the
// selection is staged in LDS and split over the 16 waves, each counting the larger keys of
// its share (and those of the key's class) from LDS broadcasts; the wave counts are summed
// in LDS and stored as the part's (rank << 16 | class rank).  Blocks past the selection's
// tiles exit at once.
__global__ __launch_bounds__(BLK) void k_nms_rank(NmsImage* __restrict__ ws) {
  __shared__ unsigned long long skey[RANK_PART];
  __shared__ int scls[RANK_PART];
  __shared__ int2 psum[BLK / 64][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int img = blockIdx.y;
  const int tile = blockIdx.x / NMS_RANK_SPLIT, part = blockIdx.x - tile * NMS_RANK_SPLIT;
  NmsImage& w = ws[img];
  const int sN = w.selN;
  if (tile >= (sN + 63) >> 6) return;   // block-uniform
  const int plen = (sN + NMS_RANK_SPLIT - 1) / NMS_RANK_SPLIT;
  const int j0 = part * plen, nj = max(0, min(sN - j0, plen));
  if (tid < nj) {
    skey[tid] = w.selKey[j0 + tid];
    scls[tid] = w.selCls[j0 + tid];
  }
  const int idx = tile * 64 + lane;
  const unsigned long long k = idx < sN ? w.selKey[idx] : ~0ull;
  const int c = idx < sN ? w.selCls[idx] : -1;
  __syncthreads();
  const int share = (nj + BLK / 64 - 1) / (BLK / 64);
  const int s0 = wave * share, s1 = min(nj, s0 + share);
  int r = 0, cr = 0;
  int j = s0;
  for (; j + 2 <= s1; j += 2) {
    const unsigned long long k0 = skey[j], k1 = skey[j + 1];
    const int c0 = scls[j], c1 = scls[j + 1];
    const bool g0 = k0 > k, g1 = k1 > k;
    r += g0 + g1;
    cr += (g0 && c0 == c) + (g1 && c1 == c);
  }
  if (j < s1) {
    const bool g0 = skey[j] > k;
    r += g0;
    cr += g0 && scls[j] == c;
  }
  psum[wave][lane] = make_int2(r, cr);
  __syncthreads();
  if (wave == 0 && idx < sN) {
    int rs = 0, crs = 0;
#pragma unroll
    for (int u = 0; u < BLK / 64; u++) {
      rs += psum[u][lane].x;
      crs += psum[u][lane].y;
    }
    w.selRank[part][idx] = ((unsigned)rs << 16) | (unsigned)crs;
  }
}

__global__ __launch_bounds__(BLK) void k_nms_layout(const int* __restrict__ counts, int A, int aux,
                                                    NmsImage* __restrict__ ws) {
  __shared__ LayoutShared L;
  const int img = blockIdx.x;
  nmsLayout(ws[img], min(min(counts[img], A), NMS_CAP), aux != 0, L);
}

// ------------------------------------------------------------------ 4. masks
// One tile (a, b) of a class per block and iteration: lane i of every wave holds member
// 64a + i (row) and member 64b + i (column); wave v tests the columns 16v .. 16v+15 (boxes
// and areas broadcast by readlane) and the four 16-bit parts meet in LDS.  On the diagonal
// only later columns count.
__global__ __launch_bounds__(256) void k_nms_masks(NmsImage* __restrict__ ws,
                                                   const PostParams* __restrict__ prm) {
  __shared__ unsigned long long part[4][64];
  const int img = blockIdx.y;
  NmsImage& w = ws[img];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nT = w.nTiles;
  const float thr = prm->iou;
  for (int it = blockIdx.x; it < nT; it += gridDim.x) {
    const int4 e = w.tile[it];
    const int cs = uni(e.x), g = uni(e.y), mo = uni(e.z), ab = uni(e.w);
    const int a = ab >> 5, b = ab & 31;
    const int row = 64 * a + lane, col = 64 * b + lane;
    const float4 rb = row < g ? w.cBox[cs + row] : make_float4(0.f, 0.f, 0.f, 0.f);
    const float4 cb = col < g ? w.cBox[cs + col] : make_float4(0.f, 0.f, 0.f, 0.f);
    const float ra = boxArea(rb), ca = boxArea(cb);
    const int j0 = 16 * wave, j1 = min(j0 + 16, g - 64 * b);
    unsigned long long word = 0ull;
    for (int j = j0; j < j1; j++) {
      const float4 bj = make_float4(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(cb.x), j)),
                                    __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cb.y), j)),
                                    __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cb.z), j)),
                                    __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cb.w), j)));
      const float baj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ca), j));
      const bool s = suppressesWave(rb, ra, bj, baj, thr);
      if ((a < b || j > lane) && s) word |= 1ull << j;
    }
    __syncthreads();   // the previous tile's parts are read
    part[wave][lane] = word;
    __syncthreads();
    if (wave == 0 && row < g)
      w.mask[mo + 32 * b * (b + 1) + row] = part[0][lane] | part[1][lane] | part[2][lane] | part[3][lane];
  }
}

// ------------------------------------------------------------------ 5. greedy
// One class per block and iteration: the block's 4 waves copy the class mask to LDS (when
// it fits GREEDY_LDS_WORDS; else the columns are read from memory), then wave 0 resolves
// the class chunk by chunk.  Lane e accumulates the members of chunk e struck by the
// survivors so far; chunk d is resolved by a bit scan over its own (diagonal) words, then
// every survivor's words for the later columns are ORed into those lanes.  The loads thus
// scale with the survivors, and the next chunk's diagonal words are fetched while the
// current one is resolved.  A class stops at max_det survivors: a later one ranks below
// max_det others.  Survivor flags are set by rank once the class is done.
__device__ __forceinline__ void greedyClass(const unsigned long long* colBase, int cs, int g, int maxdet,
                                            NmsImage& w) {
  const int lane = threadIdx.x & 63;
  const int q = (g + 63) >> 6;
  const bool later0 = lane < q;                       // lane e stands for column e
  const int laneCol = 32 * lane * (lane + 1);         // lane e's column offset
  unsigned long long struck = 0ull;                   // lane e: struck members of chunk e
  unsigned long long diagNext = lane < g ? colBase[lane] : 0ull;
  unsigned surv = 0u;                                 // bit k: this lane's member of chunk k survived
  int K = 0;
  for (int d = 0; d < q && K < maxdet; d++) {
    const unsigned long long diag = diagNext;
    if (d + 1 < q) {
      const int row = 64 * (d + 1) + lane;
      diagNext = row < g ? colBase[32 * (d + 1) * (d + 2) + row] : 0ull;
    }
    const int gq = min(64, g - 64 * d);
    unsigned long long todo = (gq >= 64 ? ~0ull : ((1ull << gq) - 1ull)) & ~readlane64(struck, d);
    unsigned long long keep = 0ull;
    while (todo) {
      const int t = __builtin_ctzll(todo);
      keep |= 1ull << t;
      todo &= ~(readlane64(diag, t) | (1ull << t));
    }
    surv |= (unsigned)((keep >> lane) & 1ull) << d;
    K += __popcll(keep);
    if (d + 1 < q && K < maxdet) {
      // survivor 64d + t strikes, in column e > d, the members of its word there
      const bool later = later0 && lane > d;
      const unsigned long long* base = colBase + laneCol + 64 * d;
      for (unsigned long long kk = keep; kk;) {
        unsigned long long v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
          const int t = kk ? __builtin_ctzll(kk) : 0;
          v[u] = (kk && later) ? base[t] : 0ull;
          kk &= kk - 1ull;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) struck |= v[u];
      }
    }
  }
  // survivor flags by rank: every chunk's rank load in flight at once
  int r[NMS_CAP / 64];
#pragma unroll
  for (int k = 0; k < NMS_CAP / 64; k++)
    if ((surv >> k) & 1u) r[k] = w.cRank[cs + 64 * k + lane];
#pragma unroll
  for (int k = 0; k < NMS_CAP / 64; k++)
    if ((surv >> k) & 1u) atomicOr(&w.kept[r[k] >> 5], 1u << (r[k] & 31));
}

__global__ __launch_bounds__(256) void k_nms_greedy(NmsImage* __restrict__ ws,
                                                    const PostParams* __restrict__ prm) {
  __shared__ unsigned long long smask[GREEDY_LDS_WORDS];
  const int img = blockIdx.y;
  NmsImage& w = ws[img];
  const int tid = threadIdx.x;
  const int P = w.nClasses;
  const int maxdet = min(prm->max_det, MAX_OUT);
  for (int it = blockIdx.x; it < P; it += gridDim.x) {
    const int4 ci = w.cls[it];
    const int cs = uni(ci.x), g = uni(ci.y), mo = uni(ci.z);
    const int q = (g + 63) >> 6;
    const int words = 32 * q * (q - 1) + g;
    const unsigned long long* src = w.mask + mo;
    const bool inLds = words <= GREEDY_LDS_WORDS;
    if (inLds) {
      __syncthreads();   // the previous class's columns are no longer read
      int i = tid;
      for (; i + 15 * 256 < words; i += 16 * 256) {
        unsigned long long v[16];
#pragma unroll
        for (int u = 0; u < 16; u++) v[u] = src[i + 256 * u];
#pragma unroll
        for (int u = 0; u < 16; u++) smask[i + 256 * u] = v[u];
      }
      for (; i < words; i += 256) smask[i] = src[i];
      __syncthreads();
    }
    if (tid < 64) {
      if (inLds) greedyClass(smask, cs, g, maxdet, w);
      else greedyClass(src, cs, g, maxdet, w);
    }
  }
}

// ------------------------------------------------------------------ 4r/5r. rotated boxes
// Suppression tiles of the rotated fast-NMS: as k_nms_masks, with probiou >= thr as the
// test.  A pair the far-pair bound rules out is skipped; the exact expression is evaluated
// as a wave-uniform branch for the lanes that need it.
__global__ __launch_bounds__(256) void k_nms_masks_obb(NmsImage* __restrict__ ws,
                                                       const PostParams* __restrict__ prm) {
  __shared__ unsigned long long part[4][64];
  const int img = blockIdx.y;
  NmsImage& w = ws[img];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nT = w.nTiles;
  const float thr = prm->iou;
  const float bstar = (thr >= 0.05f && thr <= 0.95f) ? -logf(1.f + 1e-7f - (1.f - thr) * (1.f - thr)) : 0.f;
  const float skipK = bstar > 0.f ? 8.f * bstar : INFINITY;
  auto bcast = [](float v, int j) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), j)); };
  for (int it = blockIdx.x; it < nT; it += gridDim.x) {
    const int4 e = w.tile[it];
    const int cs = uni(e.x), g = uni(e.y), mo = uni(e.z), ab = uni(e.w);
    const int a = ab >> 5, b = ab & 31;
    const int row = 64 * a + lane, col = 64 * b + lane;
    const float4 zero = make_float4(0.f, 0.f, -1.f, 0.f);
    const float4 rb = row < g ? w.cBox[cs + row] : zero, ra = row < g ? w.cAux[cs + row] : zero;
    const float4 cb = col < g ? w.cBox[cs + col] : zero, ca = col < g ? w.cAux[cs + col] : zero;
    const int j0 = 16 * wave, j1 = min(j0 + 16, g - 64 * b);
    unsigned long long word = 0ull;
    for (int j = j0; j < j1; j++) {
      const float4 bj = make_float4(bcast(cb.x, j), bcast(cb.y, j), bcast(cb.z, j), bcast(cb.w, j));
      const float4 aj = make_float4(bcast(ca.x, j), bcast(ca.y, j), bcast(ca.z, j), 0.f);
      const float dx = rb.x - bj.x, dy = rb.y - bj.y;
      const bool far = rb.z > 0.f && bj.z > 0.f && dx * dx + dy * dy > skipK * (rb.z + bj.z);
      const bool need = row < g && (a < b || j > lane) && !far;
      bool s = false;
      if (__ballot(need)) {
        if (need) s = probiou(make_float2(rb.x, rb.y), ra, rb.w, make_float2(bj.x, bj.y), aj, bj.w) >= thr;
      }
      if (s) word |= 1ull << j;
    }
    __syncthreads();   // the previous tile's parts are read
    part[wave][lane] = word;
    __syncthreads();
    if (wave == 0 && row < g)
      w.mask[mo + 32 * b * (b + 1) + row] = part[0][lane] | part[1][lane] | part[2][lane] | part[3][lane];
  }
}

// Fast-NMS decisions: one wave per (class, chunk d), taken from the diagonal tiles.  A member
// of chunk d is dropped iff some higher-ranked member of its class, suppressed or not,
// reaches it: the OR of column d's words over all its rows.  No order between chunks.
__global__ __launch_bounds__(256) void k_nms_fast(NmsImage* __restrict__ ws) {
  const int img = blockIdx.y;
  NmsImage& w = ws[img];
  const int lane = threadIdx.x & 63, wave = uni(threadIdx.x >> 6);
  const int nT = uni(w.nTiles);
  for (int it = blockIdx.x * 4 + wave; it < nT; it += gridDim.x * 4) {
    const int4 e = w.tile[it];
    const int ab = uni(e.w);
    const int d = ab & 31;
    if ((ab >> 5) != d) continue;   // wave-uniform: one diagonal tile per chunk
    const int cs = uni(e.x), g = uni(e.y), mo = uni(e.z);
    const unsigned long long* colp = w.mask + mo + 32 * d * (d + 1);
    unsigned long long v[NMS_CAP / 64];
#pragma unroll
    for (int k = 0; k < NMS_CAP / 64; k++) {
      const int row = 64 * k + lane;
      v[k] = (k <= d && row < g) ? colp[row] : 0ull;
    }
    unsigned long long dead = 0ull;
#pragma unroll
    for (int k = 0; k < NMS_CAP / 64; k++) dead |= v[k];
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) dead |= __shfl_xor(dead, o);
    const int p = 64 * d + lane;
    if (p < g && !((dead >> lane) & 1ull)) {
      const int r = w.cRank[cs + p];
      atomicOr(&w.kept[r >> 5], 1u << (r & 31));
    }
  }
}

// ------------------------------------------------------------------ 6. emit
// Thread t owns ranks 2t, 2t+1; output slots are the prefix count of survivor flags in rank
// order.  Clears the flags and re-arms the decode list for the next frame.
template <bool OBB>
__global__ __launch_bounds__(BLK) void k_nms_emit(const float* __restrict__ cand, int* __restrict__ counts,
                                                  int A, NmsImage* __restrict__ ws, float* __restrict__ out,
                                                  int* __restrict__ outidx, int* __restrict__ outcnt,
                                                  int* __restrict__ rawcnt,
                                                  const PostParams* __restrict__ prm) {
  __shared__ int wsum[BLK / 64];
  const int tid = threadIdx.x;
  const int img = blockIdx.x;
  NmsImage& w = ws[img];
  const int n = min(counts[img], A);
  const int m = min(n, NMS_CAP);
  const int maxdet = min(prm->max_det, MAX_OUT);
  const int r0 = 2 * tid, r1 = 2 * tid + 1;
  const unsigned kw = w.kept[r0 >> 5];
  const int f0 = r0 < m ? (kw >> (r0 & 31)) & 1 : 0;
  const int f1 = r1 < m ? (kw >> (r1 & 31)) & 1 : 0;
  int total;
  const int ex = blockScan<BLK>(f0 + f1, wsum, total) - f0 - f1;
  auto emit = [&](int r, int slot) {
    const int i = w.rIdx[r];
    const unsigned long long k = w.selKey[i];
    if constexpr (OBB) {   // the record as decoded: cx, cy, w, h, score, cls, theta
      const float* rec = cand + ((size_t)img * A + keyAnchor(k)) * 7;
      float* d = out + ((size_t)img * MAX_OUT + slot) * 7;
#pragma unroll
      for (int q = 0; q < 7; q++) d[q] = rec[q];
    } else {
      const float4 b = w.selBox[i];
      float* d = out + ((size_t)img * MAX_OUT + slot) * 6;
      d[0] = b.x; d[1] = b.y; d[2] = b.z; d[3] = b.w;
      d[4] = __uint_as_float((unsigned)(k >> 32));
      d[5] = (float)w.selCls[i];
    }
    outidx[img * MAX_OUT + slot] = keyAnchor(k);
  };
  if (f0 && ex < maxdet) emit(r0, ex);
  if (f1 && ex + f0 < maxdet) emit(r1, ex + f0);
  if (tid < NMS_CAP / 32) w.kept[tid] = 0u;   // every flag was read before the scan's barriers
  if (tid == 0) {
    outcnt[img] = min(total, maxdet);
    rawcnt[img] = n;
    counts[img] = 0;
  }
}

void launchNmsMulti(const float* cand, unsigned long long* lists, int* counts, int A, int cstride,
                    float* out, int* outidx, int* outcnt, int* rawcnt, const PostParams* prm,
                    NmsImage* ws, int Bn, hipStream_t st) {
  k_nms_select<false><<<Bn, BLK, 0, st>>>(cand, lists, counts, A, cstride, prm, ws);
  k_nms_rank<<<dim3(RANK_TILES * NMS_RANK_SPLIT, Bn), BLK, 0, st>>>(ws);
  k_nms_layout<<<Bn, BLK, 0, st>>>(counts, A, 0, ws);
  k_nms_masks<<<dim3(MASK_BLOCKS, Bn), 256, 0, st>>>(ws, prm);
  k_nms_greedy<<<dim3(GREEDY_BLOCKS, Bn), 256, 0, st>>>(ws, prm);
  k_nms_emit<false><<<Bn, BLK, 0, st>>>(cand, counts, A, ws, out, outidx, outcnt, rawcnt, prm);
}

void launchNmsObbMulti(const float* cand, unsigned long long* lists, int* counts, int A, float* out,
                       int* outidx, int* outcnt, int* rawcnt, const PostParams* prm, NmsImage* ws,
                       int Bn, hipStream_t st) {
  k_nms_select<true><<<Bn, BLK, 0, st>>>(cand, lists, counts, A, 7, prm, ws);
  k_nms_rank<<<dim3(RANK_TILES * NMS_RANK_SPLIT, Bn), BLK, 0, st>>>(ws);
  k_nms_layout<<<Bn, BLK, 0, st>>>(counts, A, 1, ws);
  k_nms_masks_obb<<<dim3(MASK_BLOCKS, Bn), 256, 0, st>>>(ws, prm);
  k_nms_fast<<<dim3(GREEDY_BLOCKS, Bn), 256, 0, st>>>(ws);
  k_nms_emit<true><<<Bn, BLK, 0, st>>>(cand, counts, A, ws, out, outidx, outcnt, rawcnt, prm);
}

}  // namespace yolo
