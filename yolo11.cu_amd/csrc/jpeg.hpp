// Baseline JPEG decoding split the way the hardware wants it: header parsing and entropy
// decoding (sequential within a stream) on CPU worker threads, one stream per thread, writing
// int16 coefficient planes; dequantisation, IDCT, chroma upsampling and colour conversion as
// GPU kernels over every block of a batch (jpeg.hip).  The reference server splits nvJPEG the
// same way (CPU Huffman across decoder threads, the rest on the GPU; server/serve.cpp:71-131).
//
// Supported: SOF0/SOF1 8-bit Huffman, one interleaved scan, 1 (grayscale) or 3 (YCbCr)
// components, chroma at full, half-width, half-height or half both ways, restart intervals.
// Anything else is reported unsupported so the caller can decode it another way.
#pragma once
#include <cstddef>
#include <cstdint>
#include <functional>

namespace yolo {
namespace jpeg {

struct Huff {
  uint16_t lut[512];     // next 9 bits -> length << 8 | symbol (length 0: code longer than 9)
  // AC tables: next 9 bits -> a whole (run, size, value bits) group when code and value bits
  // fit in 9 and the value in [-128, 127]: value << 8 | run << 4 | bits used; 0 otherwise
  int16_t fastAc[512];
  int32_t maxcode[18];   // largest code of each length, -1 if none; [17] is a sentinel
  int32_t valoff[17];    // symbol index of an L-bit code c = c + valoff[L]
  uint8_t sym[256];
};

struct Comp {
  int id, h, v, tq, td, ta;   // sampling factors; quantisation / DC / AC table selectors
  int cw, ch;                 // real sample-plane size
  int fh, fv;                 // upsampling factors to the luma grid (1 or 2)
  int bw, bh;                 // block grid (whole MCUs)
};

struct Header {
  int H = 0, W = 0, nc = 0, hmax = 1, vmax = 1, mcux = 0, mcuy = 0, ri = 0;
  Comp comp[3] = {};
  uint16_t q[4][64] = {};     // dequantisation tables, natural order
  bool haveQ[4] = {};
  Huff dc[4], ac[4];
  bool haveDc[4] = {}, haveAc[4] = {};
  size_t scan = 0;            // first byte of the entropy-coded segment
  size_t blocks() const {
    size_t n = 0;
    for (int c = 0; c < nc; c++) n += (size_t)comp[c].bw * comp[c].bh;
    return n;
  }
};

enum { INVALID = -1, UNSUPPORTED = 0, OK = 1 };

// Reads the markers up to the scan header: OK, UNSUPPORTED (a JPEG outside the path, or a
// frame of more than maxPixels() pixels) or INVALID (not a JPEG, or a malformed header).
int parse(const uint8_t* d, size_t n, Header& hd);

// The largest frame (height x width) parse() accepts.  A header of a few bytes can declare a
// frame of up to 65535 x 65535 pixels whose coefficients (up to 6 bytes a pixel) a decoder
// must hold, so the cap is what bounds the memory a stream can pin.  The default is PIL's
// Image.MAX_IMAGE_PIXELS (1024^3 / 4 / 3 = 89,478,485), the size above which the server's
// other decoder starts treating a frame as a decompression bomb.
constexpr long long kDefaultMaxPixels = 89478485LL;
long long maxPixels();
void setMaxPixels(long long n);

// Entropy-decodes the scan of a parsed stream into quantised coefficients, int16 in natural
// order, component plane after plane, block-row-major within a plane (hd.blocks() * 64
// values).  False on a corrupt or truncated stream.
bool decode(const uint8_t* d, size_t n, const Header& hd, int16_t* out);

// Runs fn(0 .. n-1) on the process-wide decoder threads (the calling thread helps) and
// returns when all are done.  Several threads may run loops at once.
void parallelFor(int n, const std::function<void(int)>& fn);
// Runs fn on a decoder thread; returns at once.
void runAsync(std::function<void()> fn);
int decoderThreads();

}  // namespace jpeg
}  // namespace yolo
