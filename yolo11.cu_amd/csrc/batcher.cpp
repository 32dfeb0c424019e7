// The server's batch worker, native: the reference server's per-batch loop
// (server/serve.cpp:264-302) and its deadline-aware batcher (server/serve.cpp:165-191) in C++
// on one worker thread, driving the engines only through the C ABI of include/yolo.h.  The
// caller (the gRPC front end) submits requests from any thread and collects finished ones;
// no per-batch work runs in the caller's language.
//
// Per batch, as the reference does it:
//   collect  -- the queue that is full or whose oldest request would otherwise miss the
//               target (slack = target - age - exec_ms(max batch) - stage estimate - 1 ms);
//   decode   -- JPEG streams: the entropy decoding started at submission on the library's
//               decoder threads; the coefficient copies, IDCT and colour go to the engine's
//               decode stream now, beside the previous batch's network;
//   finish   -- the previous batch: wait for it, read every slot's results into responses
//               (boxes / rotated boxes in original coordinates, top-5 classes, or boxes plus
//               RLE masks at proto resolution with the letterbox geometry);
//   stage    -- letterbox the decoded JPEG frames and stage the pixel frames (one launch);
//   launch   -- the batch graph, asynchronously.
// A stream the engine cannot decode fails only its own request; a batch that cannot be staged
// or whose results cannot be built (host allocation) fails only its own requests, and the
// worker goes on; a request the queue has no memory for is refused at submission.  A device
// failure ends the process, as everywhere in this library (engine/engine.cu:20-21).
#include <algorithm>
#include <chrono>
#include <condition_variable>
#include <cstring>
#include <deque>
#include <limits>
#include <memory>
#include <mutex>
#include <thread>
#include <vector>

#include "../../include/yolo.h"

namespace {

using Clock = std::chrono::steady_clock;
constexpr double kSafetyMs = 1.0;
constexpr int kMaxDet = 300;
constexpr int kTopK = 5;

double msSince(Clock::time_point t0, Clock::time_point t1) {
  return std::chrono::duration<double, std::milli>(t1 - t0).count();
}

struct Req {
  long long tag = 0;
  void* ticket = nullptr;               // engine-decoded JPEG, or
  const unsigned char* host = nullptr;  // R, G, B, X pixels in the caller's (pinned) memory
  int h = 0, w = 0;
  bool failed = false;
  Clock::time_point arrival;
};

struct Model {
  void* eng = nullptr;
  int maxB = 1, task = 0, mh = 0, mw = 0;
  double execMs = 0.0;
  std::deque<Req> q;
};

// A finished request: the public record plus the memory its pointers refer to.
struct Done {
  YoloBatchResult r{};
  std::vector<float> rows;
  std::vector<unsigned> rle;
  std::vector<int> rleLen;
};

struct Batch {
  int model = -1;
  std::vector<Req> reqs;
  Clock::time_point launch;
};

class Batcher {
 public:
  Batcher(void* const* engines, const int* maxB, int n, double targetMs) : targetMs_(targetMs) {
    for (int i = 0; i < n; i++) {
      Model m;
      m.eng = engines[i];
      m.maxB = std::max(1, maxB[i]);
      m.task = yolo_task(m.eng);
      m.execMs = yolo_exec_ms(m.eng, m.maxB);
      if (m.task == 3) yolo_mask_dim(m.eng, &m.mh, &m.mw);
      models_.push_back(std::move(m));
    }
    worker_ = std::thread([this] { work(); });
  }
  ~Batcher() {
    stop();
    for (Done* d : done_) delete d;   // finished and never collected
  }

  int submit(int model, Req r) {
    if (model < 0 || model >= (int)models_.size()) return -1;
    r.arrival = Clock::now();
    std::lock_guard<std::mutex> lk(mu_);
    if (stop_) return -1;
    auto& q = models_[model].q;
    try {
      q.push_back(r);
    } catch (...) {
      return -1;   // host allocation: refused like a submit after stop
    }
    // only a queue that starts (its slack now counts) or fills changes the batcher's choice
    if (q.size() == 1 || (int)q.size() >= models_[model].maxB) cv_.notify_all();
    return 0;
  }

  int wait(YoloBatchResult* out, int cap, int timeoutMs) {
    std::unique_lock<std::mutex> lk(mu_);
    auto ready = [&] { return !done_.empty() || finished_; };
    if (timeoutMs < 0) doneCv_.wait(lk, ready);
    else doneCv_.wait_for(lk, std::chrono::milliseconds(timeoutMs), ready);
    if (done_.empty()) return finished_ ? -1 : 0;
    int n = 0;
    while (n < cap && !done_.empty()) {
      Done* d = done_.front();
      done_.pop_front();
      d->r.owner = d;
      out[n++] = d->r;
    }
    return n;
  }

  // Safe from any thread and more than once: the join itself is serialised.
  void stop() {
    {
      std::lock_guard<std::mutex> lk(mu_);
      stop_ = true;
      cv_.notify_all();
    }
    std::lock_guard<std::mutex> jl(joinMu_);
    if (worker_.joinable()) worker_.join();
  }

  double stageMs() {
    std::lock_guard<std::mutex> lk(mu_);
    return stageEma_;
  }

 private:
  // The batcher's choice (server/serve.cpp:163-191): the most urgent ready queue (full, or
  // slack used up), else the queue with the least slack and how long to wait for it.
  int pick(Clock::time_point now, bool& fire, double& slackMs) const {
    int best = -1;
    fire = false;
    slackMs = std::numeric_limits<double>::infinity();
    for (int i = 0; i < (int)models_.size(); i++) {
      const Model& m = models_[i];
      if (m.q.empty()) continue;
      const double slack =
          targetMs_ - msSince(m.q.front().arrival, now) - std::max(m.execMs, 0.0) - stageEma_ - kSafetyMs;
      const bool ready = (int)m.q.size() >= m.maxB || slack <= 0;
      if ((ready && !fire) || (ready == fire && slack < slackMs)) {
        best = i;
        slackMs = slack;
        fire = fire || ready;
      }
    }
    return best;
  }

  // Blocks until a queue fires; false once stopped (queued requests are then failed).
  bool collect(Batch& b) {
    std::unique_lock<std::mutex> lk(mu_);
    for (;;) {
      if (stop_) return false;
      bool fire;
      double slack;
      const int i = pick(Clock::now(), fire, slack);
      if (i >= 0 && fire) {
        Model& m = models_[i];
        const int n = std::min((int)m.q.size(), m.maxB);
        b.model = i;
        b.reqs.assign(m.q.begin(), m.q.begin() + n);
        m.q.erase(m.q.begin(), m.q.begin() + n);
        return true;
      }
      if (i < 0) cv_.wait(lk);
      else cv_.wait_for(lk, std::chrono::microseconds((long long)(std::max(slack, 0.0) * 1000.0) + 1));
    }
  }

  // All or nothing: a range insert of pointers at the end of a deque has no effect if it
  // throws, so on failure every record is still the caller's to free.
  void publish(std::vector<Done*>& ds) {
    if (ds.empty()) return;
    std::lock_guard<std::mutex> lk(mu_);
    done_.insert(done_.end(), ds.begin(), ds.end());
    ds.clear();
    doneCv_.notify_all();
  }

  Done* failure(const Req& q, int model, int status) {
    Done* d = new Done;
    d->r.tag = q.tag;
    d->r.status = status;
    d->r.model = model;
    d->r.task = models_[model].task;
    d->r.host = q.host;
    return d;
  }

  // Reads a launched batch's results into finished requests; if that fails (host allocation),
  // the batch's requests are answered YOLO_BATCH_FAILED.
  void finish(Batch& b) {
    try {
      finishResults(b);
    } catch (...) {
      failAll(b, YOLO_BATCH_FAILED);
    }
    b.reqs.clear();
  }

  // Answers every request of a batch with `status`, releasing tickets not yet consumed.
  void failAll(Batch& b, int status) {
    std::vector<Done*> out;
    try {
      out.reserve(b.reqs.size());
      for (Req& q : b.reqs) {
        if (q.ticket) {
          yolo_jpeg_release(q.ticket);
          q.ticket = nullptr;
        }
        out.push_back(failure(q, b.model, status));
      }
      publish(out);
    } catch (...) {
      for (Done* d : out) delete d;   // nothing more can be done without memory
    }
  }

  void finishResults(Batch& b) {
    Model& m = models_[b.model];
    yolo_sync(m.eng);
    const auto now = Clock::now();
    const double inferMs = msSince(b.launch, now);
    const int B = (int)b.reqs.size();
    std::vector<YoloDet> dets;
    std::vector<YoloObbDet> obbs;
    std::vector<int> counts(B, 0);
    if (m.task == 0 || m.task == 3) {
      dets.resize((size_t)B * kMaxDet);
      yolo_get_batch(m.eng, B, dets.data(), kMaxDet, counts.data());
    } else if (m.task == 1) {
      obbs.resize((size_t)B * kMaxDet);
      yolo_get_obb_batch(m.eng, B, obbs.data(), kMaxDet, counts.data());
    }
    std::vector<unsigned char> masks;
    std::vector<Done*> out;
    try {
      out.reserve(B);   // the pushes below cannot throw: every record is freed on failure
      for (int s = 0; s < B; s++) {
        const Req& q = b.reqs[s];
        if (q.failed) {
          out.push_back(failure(q, b.model, YOLO_BATCH_DECODE_FAILED));
          continue;
        }
        Done* d = new Done;
        out.push_back(d);
        YoloBatchResult& r = d->r;
        r.tag = q.tag;
        r.model = b.model;
        r.task = m.task;
        r.batch = B;
        r.queue_ms = (float)msSince(q.arrival, b.launch);
        r.infer_ms = (float)inferMs;
        r.host = q.host;
        if (m.task == 2) {
          int ids[kTopK];
          float probs[kTopK];
          const int n = yolo_get_cls(m.eng, s, ids, probs, kTopK);
          d->rows.resize((size_t)2 * n);
          for (int j = 0; j < n; j++) {
            d->rows[2 * j] = (float)ids[j];
            d->rows[2 * j + 1] = probs[j];
          }
          r.n = n;
          r.stride = 2;
        } else if (m.task == 1) {
          const int n = counts[s];
          d->rows.resize((size_t)7 * n);
          for (int j = 0; j < n; j++) {
            const YoloObbDet& o = obbs[(size_t)s * kMaxDet + j];
            const float v[7] = {o.x, o.y, o.w, o.h, o.angle, o.score, (float)o.cls};
            std::memcpy(&d->rows[7 * j], v, sizeof v);
          }
          r.n = n;
          r.stride = 7;
        } else {
          const int n = counts[s];
          d->rows.resize((size_t)6 * n);
          for (int j = 0; j < n; j++) {
            const YoloDet& o = dets[(size_t)s * kMaxDet + j];
            const float v[6] = {o.x1, o.y1, o.x2, o.y2, o.score, (float)o.cls};
            std::memcpy(&d->rows[6 * j], v, sizeof v);
          }
          r.n = n;
          r.stride = 6;
          if (m.task == 3) {
            yolo_slot_geom(m.eng, s, &r.lb_scale, &r.lb_top, &r.lb_left);
            r.mask_h = m.mh;
            r.mask_w = m.mw;
            const size_t px = (size_t)m.mh * m.mw;
            masks.resize(px * std::max(n, 1));
            if (n > 0 && yolo_get_masks(m.eng, s, 0, n, masks.data()) != 0) std::memset(masks.data(), 0, px * n);
            d->rleLen.resize(n);
            for (int j = 0; j < n; j++) {
              // alternating 0/1 runs, row-major, starting with a 0-run (server/serve.cpp:193-203)
              const unsigned char* mk = masks.data() + px * j;
              const size_t start = d->rle.size();
              unsigned run = 0;
              bool cur = false;
              for (size_t p = 0; p < px; p++) {
                const bool v = mk[p] != 0;
                if (v != cur) {
                  d->rle.push_back(run);
                  run = 0;
                  cur = v;
                }
                run++;
              }
              d->rle.push_back(run);
              d->rleLen[j] = (int)(d->rle.size() - start);
            }
          }
        }
      }
      for (Done* d : out) {   // pointers into the vectors, now that they are final
        d->r.rows = d->rows.empty() ? nullptr : d->rows.data();
        d->r.rle = d->rle.empty() ? nullptr : d->rle.data();
        d->r.rle_len = d->rleLen.empty() ? nullptr : d->rleLen.data();
      }
      publish(out);
    } catch (...) {   // nothing of this batch was published: the caller answers all of it
      for (Done* d : out) delete d;
      throw;
    }
  }

  void work() {
    Batch prev, cur;
    bool havePrev = false;
    for (;;) {
      bool got;
      try {
        got = collect(cur);
      } catch (...) {
        // host allocation while copying a batch out of its queue: the queue is unchanged
        // (the copy comes before the erase), so its requests are taken again shortly
        cur.reqs.clear();
        std::this_thread::sleep_for(std::chrono::milliseconds(1));
        continue;
      }
      if (!got) break;
      try {
        step(prev, cur, havePrev);
      } catch (...) {
        failAll(cur, YOLO_BATCH_FAILED);   // host allocation: this batch only
        cur.reqs.clear();
      }
    }
    if (havePrev) finish(prev);
    // stopped: whatever is still queued is answered, tickets released
    for (int i = 0; i < (int)models_.size(); i++) {
      Batch left;
      left.model = i;
      {
        std::lock_guard<std::mutex> lk(mu_);
        left.reqs.assign(models_[i].q.begin(), models_[i].q.end());
        models_[i].q.clear();
      }
      failAll(left, YOLO_BATCH_STOPPED);
    }
    std::lock_guard<std::mutex> lk(mu_);
    finished_ = true;
    doneCv_.notify_all();
  }

  // One batch: decode its JPEG tickets (the previous batch still runs), answer the previous
  // batch, stage and launch this one.
  void step(Batch& prev, Batch& cur, bool& havePrev) {
    {
      Model& m = models_[cur.model];
      const auto t0 = Clock::now();
      // engine-decoded JPEG streams take the first slots, pixel frames the rest
      std::stable_partition(cur.reqs.begin(), cur.reqs.end(), [](const Req& q) { return q.ticket != nullptr; });
      const int B = (int)cur.reqs.size();
      int nj = 0;
      while (nj < B && cur.reqs[nj].ticket) nj++;
      if (nj > 0) {
        std::vector<void*> tickets(nj);
        std::vector<int> st(nj, YOLO_JPEG_INVALID);
        for (int i = 0; i < nj; i++) {
          tickets[i] = cur.reqs[i].ticket;
          cur.reqs[i].ticket = nullptr;   // consumed by the call, whatever happens
        }
        const int r = yolo_decode_tickets(m.eng, nj, tickets.data(), 0, nullptr, nullptr, st.data());
        for (int i = 0; i < nj; i++)
          if (r < 0 || st[i] != YOLO_JPEG_STAGED) cur.reqs[i].failed = true;
      }
      double stageMs = msSince(t0, Clock::now());
      if (havePrev) {
        finish(prev);
        havePrev = false;
      }
      const auto t1 = Clock::now();
      if (nj > 0) yolo_letterbox_decoded(m.eng, nj, 0);
      if (B > nj) {
        std::vector<const unsigned char*> host(B - nj);
        std::vector<int> hh(B - nj), ww(B - nj);
        for (int i = nj; i < B; i++) {
          host[i - nj] = cur.reqs[i].host;
          hh[i - nj] = cur.reqs[i].h;
          ww[i - nj] = cur.reqs[i].w;
        }
        yolo_stage_frames(m.eng, B - nj, host.data(), hh.data(), ww.data(), YOLO_PIXEL_RGBX, nj);
      }
      cur.launch = Clock::now();
      stageMs += msSince(t1, cur.launch);
      {
        std::lock_guard<std::mutex> lk(mu_);
        stageEma_ = 0.9 * stageEma_ + 0.1 * stageMs;
      }
      yolo_run_async(m.eng, B);
      std::swap(prev, cur);
      havePrev = true;
      bool idle;
      {
        std::lock_guard<std::mutex> lk(mu_);
        idle = std::all_of(models_.begin(), models_.end(), [](const Model& q) { return q.q.empty(); });
      }
      if (idle) {   // no traffic behind it: answer now
        finish(prev);
        havePrev = false;
      }
    }
  }


  std::vector<Model> models_;
  double targetMs_, stageEma_ = 1.0;
  std::mutex mu_, joinMu_;
  std::condition_variable cv_, doneCv_;
  std::deque<Done*> done_;
  bool stop_ = false, finished_ = false;
  std::thread worker_;
};

}  // namespace

void* yolo_batcher_create(void* const* engines, const int* max_batch, int n, double target_ms) {
  if (!engines || !max_batch || n < 1) return nullptr;
  for (int i = 0; i < n; i++)
    if (!engines[i]) return nullptr;
  try {
    return new Batcher(engines, max_batch, n, target_ms);
  } catch (...) {
    return nullptr;
  }
}

int yolo_batcher_submit_jpeg(void* b, int model, const unsigned char* data, size_t size, long long tag) {
  if (!b || !data) return -1;
  void* t = yolo_jpeg_submit(data, size);
  if (!t) return 1;   // not a stream the engine decodes: decode it another way
  Req r;
  r.tag = tag;
  r.ticket = t;
  if (static_cast<Batcher*>(b)->submit(model, r) != 0) {
    yolo_jpeg_release(t);
    return -1;
  }
  return 0;
}

int yolo_batcher_submit_frame(void* b, int model, const unsigned char* rgbx, int height, int width, long long tag) {
  if (!b || !rgbx || height < 1 || width < 1) return -1;
  Req r;
  r.tag = tag;
  r.host = rgbx;
  r.h = height;
  r.w = width;
  return static_cast<Batcher*>(b)->submit(model, r);
}

int yolo_batcher_wait(void* b, YoloBatchResult* out, int cap, int timeout_ms) {
  if (!b || !out || cap < 1) return -1;
  return static_cast<Batcher*>(b)->wait(out, cap, timeout_ms);
}

void yolo_batcher_release(const YoloBatchResult* r, int n) {
  for (int i = 0; r && i < n; i++) delete static_cast<Done*>(r[i].owner);
}

double yolo_batcher_stage_ms(void* b) { return b ? static_cast<Batcher*>(b)->stageMs() : -1.0; }

void yolo_batcher_stop(void* b) {
  if (b) static_cast<Batcher*>(b)->stop();
}

void yolo_batcher_destroy(void* b) { delete static_cast<Batcher*>(b); }
