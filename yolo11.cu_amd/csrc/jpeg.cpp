// JPEG headers and entropy decoding on the CPU (ITU-T T.81 Annexes B, C and F.2.2), plus the
// decoder thread pool.  Host code only.
#include "jpeg.hpp"

#include <sched.h>

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <cstdlib>
#include <deque>
#include <cstring>
#include <memory>
#include <mutex>
#include <thread>
#include <vector>

namespace yolo {
namespace jpeg {

namespace {

// zigzag position -> natural (row-major) index, T.81 Figure A.6
struct Zigzag {
  uint8_t nat[64];
  Zigzag() {
    int k = 0;
    for (int s = 0; s < 15; s++) {
      // even anti-diagonals run from bottom-left to top-right, odd ones the other way
      const int r0 = std::max(0, s - 7), r1 = std::min(7, s);
      if (s % 2 == 0)
        for (int r = r1; r >= r0; r--) nat[k++] = (uint8_t)(r * 8 + (s - r));
      else
        for (int r = r0; r <= r1; r++) nat[k++] = (uint8_t)(r * 8 + (s - r));
    }
  }
};
const Zigzag ZZ;

// Canonical code assignment (T.81 C.2) -> lookup table + per-length bounds.  False when the
// counts over-subscribe the code space.
bool buildHuff(const uint8_t* counts, const uint8_t* syms, int nsym, Huff& t) {
  std::memset(t.lut, 0, sizeof t.lut);
  std::memset(t.fastAc, 0, sizeof t.fastAc);
  std::memcpy(t.sym, syms, nsym);
  int code = 0, k = 0;
  for (int L = 1; L <= 16; L++) {
    const int c = counts[L - 1];
    t.valoff[L] = k - code;
    t.maxcode[L] = c ? code + c - 1 : -1;
    for (int i = 0; i < c; i++, k++, code++) {
      if (code >= (1 << L)) return false;
      if (L <= 9) {
        const int first = code << (9 - L), span = 1 << (9 - L);
        for (int j = 0; j < span; j++) t.lut[first + j] = (uint16_t)(L << 8 | syms[k]);
      }
    }
    code <<= 1;
  }
  t.maxcode[0] = -1;
  t.maxcode[17] = 0x7fffffff;
  // (run, size) groups whose value bits follow within the same 9-bit window
  for (int i = 0; i < 512; i++) {
    const int L = t.lut[i] >> 8, rs = t.lut[i] & 0xFF, r = rs >> 4, sz = rs & 15;
    if (L == 0 || sz == 0 || L + sz > 9) continue;
    const int bits = (i >> (9 - L - sz)) & ((1 << sz) - 1);
    const int v = bits < (1 << (sz - 1)) ? bits - (1 << sz) + 1 : bits;
    if (v >= -128 && v <= 127) t.fastAc[i] = (int16_t)(v * 256 + (r << 4) + (L + sz));
  }
  return true;
}

inline int u16(const uint8_t* p) { return p[0] << 8 | p[1]; }

// MSB-first bit reader over entropy-coded bytes: 0xFF 0x00 is a data 0xFF; at a marker (or
// the end of the data) it feeds zero bits without moving past it.
struct Bits {
  const uint8_t* d;
  size_t p, n;
  uint64_t acc = 0;   // valid bits left-aligned at bit 63
  int nb = 0;
  bool atMarker = false;

  inline void fill() {
    // fast path: whole bytes from an 8-byte window that holds no 0xFF
    if (!atMarker && p + 8 <= n) {
      uint64_t w;
      std::memcpy(&w, d + p, 8);
      const uint64_t inv = ~w;   // a 0xFF byte is a zero byte of ~w
      if (((inv - 0x0101010101010101ull) & ~inv & 0x8080808080808080ull) == 0) {
        w = __builtin_bswap64(w);
        const int k = (63 - nb) >> 3;         // bytes that fit
        if (k > 0) {
          acc |= (w >> (64 - 8 * k)) << (64 - nb - 8 * k);
          nb += 8 * k;
          p += k;
        }
        return;
      }
    }
    while (nb <= 56) {
      uint64_t b = 0;
      if (!atMarker && p < n) {
        b = d[p];
        if (b == 0xFF) {
          const uint8_t nx = p + 1 < n ? d[p + 1] : 0xD9;
          if (nx == 0x00) {
            p += 2;
          } else {
            atMarker = true;
            b = 0;
          }
        } else {
          p++;
        }
      }
      acc |= b << (56 - nb);
      nb += 8;
    }
  }
  inline uint32_t peek(int k) const { return (uint32_t)(acc >> (64 - k)); }
  inline void skip(int k) {
    acc <<= k;
    nb -= k;
  }
  // s (<= 16) raw bits, sign-extended per EXTEND (F.2.2.1)
  inline int receiveExtend(int s) {
    if (s == 0) return 0;
    const int v = (int)peek(s);
    skip(s);
    return v < (1 << (s - 1)) ? v - (1 << s) + 1 : v;
  }
  // Huffman symbol, or -1 on an invalid code
  inline int decode(const Huff& t) {
    const uint16_t e = t.lut[peek(9)];
    if (e >> 8) {
      skip(e >> 8);
      return e & 0xFF;
    }
    const uint32_t c16 = peek(16);
    for (int L = 10; L <= 16; L++) {
      const int c = (int)(c16 >> (16 - L));
      if (c <= t.maxcode[L]) {
        skip(L);
        const int i = c + t.valoff[L];
        return i >= 0 && i < 256 ? t.sym[i] : -1;
      }
    }
    return -1;
  }
  // end of a restart interval: drop the partial byte and step over RSTn
  void restart() {
    acc = 0;
    nb = 0;
    atMarker = false;
    while (p + 1 < n && d[p] == 0xFF && d[p + 1] == 0xFF) p++;
    if (p + 1 < n && d[p] == 0xFF && d[p + 1] >= 0xD0 && d[p + 1] <= 0xD7) p += 2;
  }
};

// ------------------------------------------------------------------ decoder threads
// A queue of tasks served by the decoder threads.  A parallel-for posts helper tasks that pull
// indices from a shared counter, and the caller pulls too; a helper that starts after the
// loop is done finds the counter exhausted and never touches the loop's function.
class Pool {
 public:
  explicit Pool(int workers) {
    for (int i = 0; i < workers; i++) th_.emplace_back([this] { loop(); });
  }
  int size() const { return (int)th_.size() + 1; }

  void post(std::function<void()> f) {
    {
      std::lock_guard<std::mutex> lk(mu_);
      q_.push_back(std::move(f));
    }
    cv_.notify_one();
  }

  void run(int n, const std::function<void(int)>& fn) {
    auto job = std::make_shared<Job>();
    job->fn = &fn;
    job->n = n;
    const int helpers = std::min(n - 1, (int)th_.size());
    for (int i = 0; i < helpers; i++) post([job] { job->work(); });
    job->work();
    std::unique_lock<std::mutex> lk(job->mu);
    job->cv.wait(lk, [&] { return job->done.load() == job->n; });
  }

 private:
  struct Job {
    const std::function<void(int)>* fn = nullptr;
    int n = 0;
    std::atomic<int> next{0}, done{0};
    std::mutex mu;
    std::condition_variable cv;
    void work() {
      for (;;) {
        const int i = next.fetch_add(1);
        if (i >= n) return;
        (*fn)(i);
        if (done.fetch_add(1) + 1 == n) {
          std::lock_guard<std::mutex> lk(mu);
          cv.notify_all();
        }
      }
    }
  };

  void loop() {
    for (;;) {
      std::function<void()> f;
      {
        std::unique_lock<std::mutex> lk(mu_);
        cv_.wait(lk, [&] { return !q_.empty(); });
        f = std::move(q_.front());
        q_.pop_front();
      }
      f();
    }
  }

  std::vector<std::thread> th_;
  std::mutex mu_;
  std::condition_variable cv_;
  std::deque<std::function<void()>> q_;
};

int threadCount() {
  if (const char* s = std::getenv("YOLO_DECODE_THREADS")) {
    const int v = std::atoi(s);
    if (v >= 1) return std::min(v, 256);
  }
  cpu_set_t set;
  int n = 8;
  if (sched_getaffinity(0, sizeof set, &set) == 0) n = CPU_COUNT(&set);
  return std::max(1, std::min(n, 16));
}

Pool& pool() {
  // never destroyed: the workers wait on their condition variable until the process ends
  static Pool* p = new Pool(threadCount() - 1);
  return *p;
}

}  // namespace

int decoderThreads() { return pool().size(); }

void parallelFor(int n, const std::function<void(int)>& fn) {
  if (n <= 0) return;
  if (n == 1) {
    fn(0);
    return;
  }
  pool().run(n, fn);
}

void runAsync(std::function<void()> fn) { pool().post(std::move(fn)); }

// ------------------------------------------------------------------ headers
namespace {
std::atomic<long long> g_maxPixels{kDefaultMaxPixels};
}  // namespace

long long maxPixels() { return g_maxPixels.load(std::memory_order_relaxed); }
void setMaxPixels(long long n) { g_maxPixels.store(n, std::memory_order_relaxed); }

int parse(const uint8_t* d, size_t n, Header& hd) {
  if (n < 4 || d[0] != 0xFF || d[1] != 0xD8) return INVALID;
  bool haveFrame = false, jfif = false;
  int adobe = -1;
  size_t p = 2;
  while (p + 4 <= n) {
    if (d[p] != 0xFF) return INVALID;
    const int m = d[p + 1];
    if (m == 0xFF) {
      p++;
      continue;
    }
    if (m == 0xD8 || m == 0x01 || (m >= 0xD0 && m <= 0xD7)) {   // no length field
      p += 2;
      continue;
    }
    if (m == 0xD9) return INVALID;         // end of image before any scan
    const int len = u16(d + p + 2);
    if (len < 2 || p + 2 + len > n) return INVALID;
    const uint8_t* s = d + p + 4;
    const int sl = len - 2;
    if (m == 0xC0 || m == 0xC1) {
      if (sl < 6) return INVALID;
      if (s[0] != 8) return UNSUPPORTED;
      hd.H = u16(s + 1);
      hd.W = u16(s + 3);
      hd.nc = s[5];
      if (hd.nc != 1 && hd.nc != 3) return UNSUPPORTED;
      if (sl < 6 + 3 * hd.nc) return INVALID;
      for (int c = 0; c < hd.nc; c++) {
        Comp& k = hd.comp[c];
        k.id = s[6 + 3 * c];
        k.h = s[7 + 3 * c] >> 4;
        k.v = s[7 + 3 * c] & 15;
        k.tq = s[8 + 3 * c];
        if (k.h < 1 || k.h > 4 || k.v < 1 || k.v > 4 || k.tq > 3) return INVALID;
      }
      haveFrame = true;
    } else if ((m >= 0xC2 && m <= 0xCF) && m != 0xC4 && m != 0xC8 && m != 0xCC) {
      return UNSUPPORTED;                  // progressive, lossless, arithmetic, hierarchical
    } else if (m == 0xC4) {
      int i = 0;
      while (i < sl) {
        if (i + 17 > sl) return INVALID;
        const int tc = s[i] >> 4, th = s[i] & 15;
        if (tc > 1 || th > 3) return INVALID;
        int nsym = 0;
        for (int L = 0; L < 16; L++) nsym += s[i + 1 + L];
        if (nsym > 256 || i + 17 + nsym > sl) return INVALID;
        Huff& t = tc == 0 ? hd.dc[th] : hd.ac[th];
        if (!buildHuff(s + i + 1, s + i + 17, nsym, t)) return INVALID;
        (tc == 0 ? hd.haveDc : hd.haveAc)[th] = true;
        i += 17 + nsym;
      }
    } else if (m == 0xDB) {
      int i = 0;
      while (i < sl) {
        const int pq = s[i] >> 4, tq = s[i] & 15;
        if (tq > 3 || pq > 1 || i + 1 + 64 * (pq + 1) > sl) return INVALID;
        for (int k = 0; k < 64; k++)
          hd.q[tq][ZZ.nat[k]] = (uint16_t)(pq ? u16(s + i + 1 + 2 * k) : s[i + 1 + k]);
        hd.haveQ[tq] = true;
        i += 1 + 64 * (pq + 1);
      }
    } else if (m == 0xDD) {
      if (sl < 2) return INVALID;
      hd.ri = u16(s);
    } else if (m == 0xE0 && sl >= 5 && std::memcmp(s, "JFIF\0", 5) == 0) {
      jfif = true;
    } else if (m == 0xEE && sl >= 12 && std::memcmp(s, "Adobe", 5) == 0) {
      adobe = s[11];
    } else if (m == 0xDA) {
      if (!haveFrame || sl < 1) return INVALID;
      const int ns = s[0];
      if (sl < 4 + 2 * ns) return INVALID;
      if (ns != hd.nc) return UNSUPPORTED;  // one interleaved scan (or the one component)
      for (int c = 0; c < ns; c++) {
        if (s[1 + 2 * c] != hd.comp[c].id) return UNSUPPORTED;
        hd.comp[c].td = s[2 + 2 * c] >> 4;
        hd.comp[c].ta = s[2 + 2 * c] & 15;
        if (hd.comp[c].td > 3 || hd.comp[c].ta > 3) return INVALID;
        if (!hd.haveDc[hd.comp[c].td] || !hd.haveAc[hd.comp[c].ta] || !hd.haveQ[hd.comp[c].tq]) return INVALID;
      }
      if (s[1 + 2 * ns] != 0 || s[2 + 2 * ns] != 63 || s[3 + 2 * ns] != 0) return UNSUPPORTED;
      hd.scan = p + 2 + len;
      // colour space as libjpeg infers it: JFIF -> YCbCr; else the Adobe transform flag
      // (0 = RGB); else component ids 'R','G','B' -> RGB.  RGB streams take the other path.
      if (hd.nc == 3 && !jfif) {
        const bool rgb = adobe >= 0 ? adobe == 0
                                    : (hd.comp[0].id == 'R' && hd.comp[1].id == 'G' && hd.comp[2].id == 'B');
        if (rgb) return UNSUPPORTED;
      }
      if (hd.H < 1 || hd.W < 1 || (long long)hd.H * hd.W > maxPixels()) return UNSUPPORTED;
      hd.hmax = hd.vmax = 1;
      for (int c = 0; c < hd.nc; c++) {
        hd.hmax = std::max(hd.hmax, hd.comp[c].h);
        hd.vmax = std::max(hd.vmax, hd.comp[c].v);
      }
      for (int c = 0; c < hd.nc; c++) {
        Comp& k = hd.comp[c];
        if (hd.nc == 1) {
          k.fh = k.fv = 1;
          k.cw = hd.W;
          k.ch = hd.H;
          k.bw = (hd.W + 7) / 8;
          k.bh = (hd.H + 7) / 8;
          continue;
        }
        if (hd.hmax % k.h || hd.vmax % k.v) return UNSUPPORTED;
        k.fh = hd.hmax / k.h;
        k.fv = hd.vmax / k.v;
        if (k.fh > 2 || k.fv > 2 || (c == 0 && (k.fh != 1 || k.fv != 1))) return UNSUPPORTED;
        k.cw = (int)(((long)hd.W * k.h + hd.hmax - 1) / hd.hmax);
        k.ch = (int)(((long)hd.H * k.v + hd.vmax - 1) / hd.vmax);
        if ((k.fh == 2 && k.cw < 3) || (k.fv == 2 && k.ch < 3)) return UNSUPPORTED;
      }
      if (hd.nc == 3) {
        hd.mcux = (hd.W + 8 * hd.hmax - 1) / (8 * hd.hmax);
        hd.mcuy = (hd.H + 8 * hd.vmax - 1) / (8 * hd.vmax);
        for (int c = 0; c < 3; c++) {
          hd.comp[c].bw = hd.mcux * hd.comp[c].h;
          hd.comp[c].bh = hd.mcuy * hd.comp[c].v;
        }
      } else {
        hd.mcux = hd.comp[0].bw;
        hd.mcuy = hd.comp[0].bh;
      }
      return OK;
    }
    p += 2 + len;
  }
  return INVALID;
}

// ------------------------------------------------------------------ entropy decoding
bool decode(const uint8_t* d, size_t n, const Header& hd, int16_t* out) {
  Bits b{d, hd.scan, n};
  int16_t* plane[3];
  size_t off = 0;
  for (int c = 0; c < hd.nc; c++) {
    plane[c] = out + off * 64;
    off += (size_t)hd.comp[c].bw * hd.comp[c].bh;
  }
  int pred[3] = {0, 0, 0};

  auto block = [&](int c, int by, int bx) -> bool {
    const Comp& k = hd.comp[c];
    int16_t* blk = plane[c] + ((size_t)by * k.bw + bx) * 64;
    std::memset(blk, 0, 64 * sizeof(int16_t));
    b.fill();
    const int s = b.decode(hd.dc[k.td]);
    if (s < 0 || s > 15) return false;
    pred[c] += b.receiveExtend(s);
    blk[0] = (int16_t)pred[c];
    const Huff& ac = hd.ac[k.ta];
    for (int i = 1; i < 64;) {
      if (b.nb < 32) b.fill();
      const int fa = ac.fastAc[b.peek(9)];
      if (fa) {                             // code, run and value in one lookup
        b.skip(fa & 15);
        i += (fa >> 4) & 15;
        if (i > 63) return false;
        blk[ZZ.nat[i]] = (int16_t)(fa >> 8);
        i++;
        continue;
      }
      const int rs = b.decode(ac);
      if (rs < 0) return false;
      const int r = rs >> 4, sz = rs & 15;
      if (sz == 0) {
        if (r != 15) break;                 // end of block
        i += 16;
        continue;
      }
      i += r;
      if (i > 63) return false;
      blk[ZZ.nat[i]] = (int16_t)b.receiveExtend(sz);
      i++;
    }
    return true;
  };

  const long mcus = (long)hd.mcux * hd.mcuy;
  for (long m = 0; m < mcus; m++) {
    if (hd.ri && m && m % hd.ri == 0) {
      b.restart();
      pred[0] = pred[1] = pred[2] = 0;
    }
    const int my = (int)(m / hd.mcux), mx = (int)(m % hd.mcux);
    if (hd.nc == 1) {
      if (!block(0, my, mx)) return false;
      continue;
    }
    for (int c = 0; c < hd.nc; c++) {
      const Comp& k = hd.comp[c];
      for (int y = 0; y < k.v; y++)
        for (int x = 0; x < k.h; x++)
          if (!block(c, my * k.v + y, mx * k.h + x)) return false;
    }
  }
  // the scan ended on a marker (EOI, normally); running off the end of the data is a
  // truncated stream
  return b.p < n;
}

}  // namespace jpeg
}  // namespace yolo
