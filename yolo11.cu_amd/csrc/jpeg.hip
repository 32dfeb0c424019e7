// The GPU half of the JPEG decode: dequantisation + IDCT of every block of a batch, then chroma
// upsampling + YCbCr -> RGB per pixel into R, G, B, X frames that the letterbox reads.  Integer
// arithmetic throughout, so the samples equal the CPU decoder's (PIL / libjpeg-turbo) exactly:
// the "islow" IDCT (13-bit constants, rounding shifts, range limit), "fancy" triangle-filter
// upsampling and 16-bit fixed-point colour conversion.
#include "engine.hpp"

namespace yolo {

namespace {

// 13-bit fixed-point multipliers, round(x * 2^13)
constexpr int fix13(double x) { return (int)(x * 8192 + 0.5); }
constexpr int F0298 = fix13(0.298631336), F0390 = fix13(0.390180644), F0541 = fix13(0.541196100),
              F0765 = fix13(0.765366865), F0899 = fix13(0.899976223), F1175 = fix13(1.175875602),
              F1501 = fix13(1.501321110), F1847 = fix13(1.847759065), F1961 = fix13(1.961570560),
              F2053 = fix13(2.053119869), F2562 = fix13(2.562915447), F3072 = fix13(3.072711026);
// 16-bit fixed-point colour multipliers, round(x * 2^16)
constexpr int fix16(double x) { return (int)(x * 65536 + 0.5); }
constexpr int CR_R = fix16(1.40200), CB_B = fix16(1.77200), CR_G = fix16(0.71414), CB_G = fix16(0.34414);

// One 8-point pass (Loeffler-Ligtenberg-Moschytz, as in the IJG islow IDCT): x[k] is the k-th
// frequency term, o[n] the n-th sample, rounded right shift by `shift`.
__device__ __forceinline__ void idct8(const int* x, int* o, int shift) {
  int z1 = (x[2] + x[6]) * F0541;
  const int t2 = z1 - x[6] * F1847;
  const int t3 = z1 + x[2] * F0765;
  const int t0 = (x[0] + x[4]) << 13;
  const int t1 = (x[0] - x[4]) << 13;
  const int e10 = t0 + t3, e13 = t0 - t3, e11 = t1 + t2, e12 = t1 - t2;
  int a0 = x[7], a1 = x[5], a2 = x[3], a3 = x[1];
  z1 = a0 + a3;
  int z2 = a1 + a2, z3 = a0 + a2, z4 = a1 + a3;
  const int z5 = (z3 + z4) * F1175;
  a0 *= F0298;
  a1 *= F2053;
  a2 *= F3072;
  a3 *= F1501;
  z1 *= -F0899;
  z2 *= -F2562;
  z3 = z3 * -F1961 + z5;
  z4 = z4 * -F0390 + z5;
  a0 += z1 + z3;
  a1 += z2 + z4;
  a2 += z2 + z3;
  a3 += z1 + z4;
  const int r = 1 << (shift - 1);
  o[0] = (e10 + a3 + r) >> shift;
  o[7] = (e10 - a3 + r) >> shift;
  o[1] = (e11 + a2 + r) >> shift;
  o[6] = (e11 - a2 + r) >> shift;
  o[2] = (e12 + a1 + r) >> shift;
  o[5] = (e12 - a1 + r) >> shift;
  o[3] = (e13 + a0 + r) >> shift;
  o[4] = (e13 - a0 + r) >> shift;
}

// The post-IDCT range limit: v + 128 clamped to [0, 255] for v in [-128, 511], with the
// table's wrap (index v & 1023) beyond that.
__device__ __forceinline__ uint32_t rangeLimit(int v) {
  const int w = v & 1023;
  return (uint32_t)(w < 128 ? w + 128 : w < 512 ? 255 : w < 896 ? 0 : w - 896);
}

constexpr int IDCT_BLOCKS = 32;   // 8 lanes per block, 256 threads

// grid: ceil(nblocks / 32).  Lane c of a block runs the column pass on column c, then the
// row pass on row c, and stores that row's 8 samples with one 8-byte store.
__global__ __launch_bounds__(256) void k_jpeg_idct(const int16_t* __restrict__ coef,
                                                   const JpegPlane* __restrict__ planes, int nplanes,
                                                   int nblocks, uint8_t* __restrict__ samples) {
  __shared__ int ws[IDCT_BLOCKS][8][9];
  const int lb = threadIdx.x >> 3, c = threadIdx.x & 7;
  const int gb = blockIdx.x * IDCT_BLOCKS + lb;
  const bool live = gb < nblocks;
  int lo = 0, hi = nplanes - 1;           // last plane whose first block is <= gb
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if ((int)planes[mid].block0 <= gb) lo = mid;
    else hi = mid - 1;
  }
  const JpegPlane& P = planes[lo];
  int x[8], o[8];
  const int16_t* cb = coef + (size_t)(live ? gb : 0) * 64;
#pragma unroll
  for (int u = 0; u < 8; u++) x[u] = live ? (int)cb[u * 8 + c] * (int)P.q[u * 8 + c] : 0;
  idct8(x, o, 11);                        // 13 - 2 bits: two extra bits kept for the row pass
#pragma unroll
  for (int y = 0; y < 8; y++) ws[lb][y][c] = o[y];
  __syncthreads();
#pragma unroll
  for (int v = 0; v < 8; v++) x[v] = ws[lb][c][v];
  idct8(x, o, 18);                        // 13 + 2 + 3 bits
  const int local = gb - (int)P.block0;   // blocks of streams that failed to decode lie in
  if (!live || local < 0 || local >= (int)P.bw * (int)P.bh) return;   // no plane: skipped
  const uint32_t lo4 = rangeLimit(o[0]) | rangeLimit(o[1]) << 8 | rangeLimit(o[2]) << 16 | rangeLimit(o[3]) << 24;
  const uint32_t hi4 = rangeLimit(o[4]) | rangeLimit(o[5]) << 8 | rangeLimit(o[6]) << 16 | rangeLimit(o[7]) << 24;
  const int by = local / P.bw, bx = local - by * P.bw;
  uint8_t* dst = samples + P.out + (size_t)(by * 8 + c) * (P.bw * 8) + bx * 8;
  *reinterpret_cast<uint2*>(dst) = make_uint2(lo4, hi4);
}

// Chroma sample at luma position (x, y) of a plane subsampled by (fh, fv): the triangle
// ("fancy") filters with their alternating rounding biases, edge columns special-cased and
// the neighbouring row clamped to the real plane.
__device__ __forceinline__ int chroma(const uint8_t* __restrict__ p, int stride, int cw, int ch, int fh, int fv,
                                      int x, int y) {
  const int cx = fh == 2 ? x >> 1 : x, cy = fv == 2 ? y >> 1 : y;
  const uint8_t* row = p + (size_t)cy * stride;
  if (fv == 1) {
    if (fh == 1) return row[cx];
    if ((x & 1) == 0) return cx == 0 ? row[0] : (3 * row[cx] + row[cx - 1] + 1) >> 2;
    return cx == cw - 1 ? row[cx] : (3 * row[cx] + row[cx + 1] + 2) >> 2;
  }
  const bool lower = y & 1;
  const uint8_t* nb = p + (size_t)(lower ? min(cy + 1, ch - 1) : max(cy - 1, 0)) * stride;
  if (fh == 1) return (3 * row[cx] + nb[cx] + (lower ? 2 : 1)) >> 2;
  const int s = 3 * row[cx] + nb[cx];
  if ((x & 1) == 0) return cx == 0 ? (4 * s + 8) >> 4 : (3 * s + 3 * row[cx - 1] + nb[cx - 1] + 8) >> 4;
  return cx == cw - 1 ? (4 * s + 7) >> 4 : (3 * s + 3 * row[cx + 1] + nb[cx + 1] + 7) >> 4;
}

__device__ __forceinline__ uint32_t clamp255(int v) { return (uint32_t)min(max(v, 0), 255); }

// grid (ceil(max pixels / 256), images): one thread per output pixel.
__global__ __launch_bounds__(256) void k_jpeg_color(const uint8_t* __restrict__ samples,
                                                    const JpegFrame* __restrict__ frames) {
  const JpegFrame& F = frames[blockIdx.y];
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= F.H * F.W) return;
  const int y = idx / F.W, x = idx - y * F.W;
  const int Y = samples[F.plane[0] + (size_t)y * F.stride[0] + x];
  uint32_t px;
  if (F.nc == 1) {
    px = (uint32_t)Y * 0x010101u | 0xFF000000u;
  } else {
    const int cb = chroma(samples + F.plane[1], F.stride[1], F.cw[1], F.ch[1], F.fh[1], F.fv[1], x, y) - 128;
    const int cr = chroma(samples + F.plane[2], F.stride[2], F.cw[2], F.ch[2], F.fh[2], F.fv[2], x, y) - 128;
    const uint32_t r = clamp255(Y + ((CR_R * cr + 32768) >> 16));
    const uint32_t g = clamp255(Y + ((-CB_G * cb + 32768 - CR_G * cr) >> 16));
    const uint32_t b = clamp255(Y + ((CB_B * cb + 32768) >> 16));
    px = r | g << 8 | b << 16 | 0xFF000000u;
  }
  reinterpret_cast<uint32_t*>(F.dst)[idx] = px;
}

}  // namespace

void launchJpegIdct(const int16_t* coef, const JpegPlane* planes, int nplanes, int nblocks, uint8_t* samples,
                    hipStream_t st) {
  if (nblocks <= 0 || nplanes <= 0) return;
  k_jpeg_idct<<<(nblocks + IDCT_BLOCKS - 1) / IDCT_BLOCKS, 256, 0, st>>>(coef, planes, nplanes, nblocks, samples);
}

void launchJpegColor(const uint8_t* samples, const JpegFrame* frames, int nframes, int maxPixels, hipStream_t st) {
  if (nframes <= 0 || maxPixels <= 0) return;
  k_jpeg_color<<<dim3((maxPixels + 255) / 256, nframes), 256, 0, st>>>(samples, frames);
}

}  // namespace yolo
