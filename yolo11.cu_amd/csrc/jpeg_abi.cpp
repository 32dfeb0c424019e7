// The host-only JPEG entry points of include/yolo.h.  Built into the engine library and, alone
// with jpeg.cpp, into libyolo11_jpeg.so: a library without the HIP runtime that a process which
// must not touch the GPU (a server front-end) can load to read JPEG headers.
#include "../../include/yolo.h"
#include "jpeg.hpp"

// No exception leaves these functions: a host allocation (or thread creation) failure reads
// as an error code.
int yolo_jpeg_probe(const unsigned char* data, size_t size, int* height, int* width) {
  if (!data) return -1;
  try {
    yolo::jpeg::Header hd;
    const int r = yolo::jpeg::parse(data, size, hd);
    if (r == yolo::jpeg::OK) {
      if (height) *height = hd.H;
      if (width) *width = hd.W;
    }
    return r;
  } catch (...) {
    return -1;
  }
}

int yolo_decoder_threads(void) {
  try {
    return yolo::jpeg::decoderThreads();
  } catch (...) {
    return -1;
  }
}

long long yolo_jpeg_max_pixels(long long n) {
  if (n > 0) yolo::jpeg::setMaxPixels(n);
  return yolo::jpeg::maxPixels();
}

long long yolo_jpeg_coefficients(const unsigned char* data, size_t size, short* out, size_t cap) {
  if (!data) return -1;
  try {
    yolo::jpeg::Header hd;
    if (yolo::jpeg::parse(data, size, hd) != yolo::jpeg::OK) return -1;
    const size_t n = hd.blocks() * 64;
    if (!out) return (long long)n;
    if (cap < n) return -1;
    return yolo::jpeg::decode(data, size, hd, out) ? (long long)n : -2;
  } catch (...) {
    return -1;
  }
}
