// producer.cpp -- host CPU shards running SSLA-S stages 0 + 1 and feeding the
// drain's rings: libstage01_to_gpu.so (s01g_*) and libstage01_capi.so (s0_*).
//
// Threads: one submitting thread (s01g_submit_batch, or the synthetic source)
// routes each event to the x-strip shards that need it through per-shard
// single-producer / single-consumer queues; every shard thread owns a private
// Stage01 state.  The owner shard of an event runs the stages and, in the GPU
// library, publishes surviving records to the attached rings.
//
// Build-time switch: STAGE01_TO_GPU selects the s01g_* library (tdrop checked
// before the stages so dropped work runs state-only, and ring publishing);
// without it the file builds the s0_* library (full stage 0 for every event,
// tdrops after the stages, as the CPU-only reference path does).
#include <pthread.h>
#include <sched.h>
#include <time.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <exception>
#include <memory>
#include <random>
#include <thread>
#include <vector>

#include "ssla_abi.h"
#include "stage01.h"

namespace ssla {
namespace {

std::uint64_t mono_ns() {
    timespec ts;
    clock_gettime(CLOCK_MONOTONIC_RAW, &ts);
    return (std::uint64_t)ts.tv_sec * 1000000000ull + (std::uint64_t)ts.tv_nsec;
}

void pin_self(int core) {
    if (core < 0) return;
    const unsigned n = std::thread::hardware_concurrency();
    if (n && (unsigned)core >= n) return;
    cpu_set_t cs;
    CPU_ZERO(&cs);
    CPU_SET(core, &cs);
    pthread_setaffinity_np(pthread_self(), sizeof(cs), &cs);
}

inline void cpu_relax() { __builtin_ia32_pause(); }

// Bounded single-producer / single-consumer queue (capacity 2^k).
template <class T>
class Queue {
public:
    explicit Queue(std::size_t cap) : mask_(cap - 1), buf_(cap) {}
    bool try_push(const T& v) {
        const std::size_t h = head_.load(std::memory_order_relaxed);
        if (h - tail_.load(std::memory_order_acquire) > mask_) return false;
        buf_[h & mask_] = v;
        head_.store(h + 1, std::memory_order_release);
        return true;
    }
    void push(const T& v) {
        while (!try_push(v)) cpu_relax();
    }
    bool try_pop(T& out) {
        const std::size_t t = tail_.load(std::memory_order_relaxed);
        if (t == head_.load(std::memory_order_acquire)) return false;
        out = buf_[t & mask_];
        tail_.store(t + 1, std::memory_order_release);
        return true;
    }
    std::size_t size() const {
        return head_.load(std::memory_order_relaxed) - tail_.load(std::memory_order_relaxed);
    }

private:
    const std::size_t mask_;
    std::vector<T> buf_;
    alignas(64) std::atomic<std::size_t> head_{0};
    alignas(64) std::atomic<std::size_t> tail_{0};
};

struct Msg {
    std::uint64_t t_arr_ns;    // entered the shard queue
    std::uint64_t t_emit_ns;   // produced by the source
    float t, x, y, p;
    std::uint8_t owner, eof;
};

enum Seg { SEG_PRE, SEG_S0, SEG_TD0, SEG_S1, SEG_TD1, SEG_PUSH, NSEG };

struct Shard {
    int id = 0, core = -1;
    std::unique_ptr<Stage01> st;
    std::unique_ptr<Queue<Msg>> q;
    std::vector<double> samples;
    std::atomic<std::size_t> n_samples{0};
    std::atomic<std::uint64_t> owner{0}, halo{0}, pass0{0}, pass1{0};
    std::atomic<std::uint64_t> seg_ns[NSEG] = {}, seg_n[NSEG] = {};
};

struct RingOut {
    HybridInputRec* buf = nullptr;
    std::uint64_t* head = nullptr;
    const std::uint64_t* tail = nullptr;   // consumer's tail (back-pressure), or null
    int x_lo = 0, x_hi = 0, y_lo = 0, y_hi = 0;
    std::atomic<std::uint64_t> pushed{0};
};

constexpr int kMaxRings = SSLA_MAX_BLOCKS;

}  // namespace

struct Producer {
    int N = 1, halo = 2, strip = 1, W = 0, H = 0;
    std::vector<std::unique_ptr<Shard>> shards;
    std::vector<std::thread> threads;
    std::atomic<std::uint64_t> oob{0};
    std::chrono::steady_clock::time_point t0;
    // rings
    std::atomic<bool> attached{false};
    RingOut rings[kMaxRings];
    int n_rings = 0, W2 = 0, H2 = 0;
    std::uint64_t ring_mask = 0;
    // back-pressure: a claimed slot waits for the consumer's tail to free it
    std::uint64_t bp_timeout_ns = 0;
    std::atomic<std::uint64_t> bp_waits{0}, bp_wait_ns{0}, bp_overruns{0};
    // synthetic source
    std::atomic<bool> synth_on{false};
    std::thread synth;
    std::atomic<std::uint64_t> synth_n{0};

    // now: the enqueue time (0: read the clock here)
    void route(float t, float x, float y, float p, std::uint64_t t_emit, std::uint64_t now = 0) {
        const int ex = (int)x, ey = (int)y;
        if (ex < 0 || ex >= W || ey < 0 || ey >= H) {
            oob.fetch_add(1, std::memory_order_relaxed);
            return;
        }
        const int home = ex / strip;
        const int owner = std::min(home, N - 1);
        if (now == 0) now = mono_ns();
        for (int k = std::max(0, home - 1); k <= std::min(N - 1, home + 1); ++k) {
            if (ex < k * strip - halo || ex >= (k + 1) * strip + halo) continue;
            Msg m{now, t_emit, t, x, y, p, (std::uint8_t)(k == owner), 0};
            shards[k]->q->push(m);
        }
    }

    void publish(int x2, int y2, float t, const float* feat1, std::uint64_t t_emit) {
        if (x2 < 0 || x2 >= W2 || y2 < 0 || y2 >= H2) return;
        for (int b = 0; b < n_rings; ++b) {
            RingOut& r = rings[b];
            if (x2 < r.x_lo || x2 >= r.x_hi || y2 < r.y_lo || y2 >= r.y_hi) continue;
            const std::uint64_t slot = __atomic_fetch_add(r.head, 1ull, __ATOMIC_RELAXED);
            if (r.tail && slot - __atomic_load_n(r.tail, __ATOMIC_ACQUIRE) > ring_mask) {
                // the slot still holds a record the consumer has not taken:
                // wait for it, up to bp_timeout_ns, then overwrite (the
                // consumer reports the overrun)
                const std::uint64_t w0 = mono_ns();
                std::uint64_t now = w0;
                while (slot - __atomic_load_n(r.tail, __ATOMIC_ACQUIRE) > ring_mask) {
                    cpu_relax();
                    now = mono_ns();
                    if (now - w0 > bp_timeout_ns) {
                        bp_overruns.fetch_add(1, std::memory_order_relaxed);
                        break;
                    }
                }
                bp_waits.fetch_add(1, std::memory_order_relaxed);
                bp_wait_ns.fetch_add(now - w0, std::memory_order_relaxed);
            }
            HybridInputRec* d = r.buf + (slot & ring_mask);
            d->t = t;
            d->x = (unsigned short)x2;
            d->y = (unsigned short)y2;
            std::memcpy(d->feat1, feat1, sizeof(float) * SSLA_C1);
            d->t_push_ns = mono_ns();
            d->t_emit_ns = t_emit;
            __atomic_store_n(&d->seq_done, slot + 1ull, __ATOMIC_RELEASE);
            r.pushed.fetch_add(1, std::memory_order_relaxed);
        }
    }

    // Shard loop: takes what its queue holds (up to kBatch messages, never
    // waiting for more), decides tdrop for each message in order, then runs
    // the stages layer by layer over the batch (Stage01::stage*_batch; each
    // layer's state still sees the events in queue order) and publishes the
    // pass-1 records in order.  A message's segment times are its batch's
    // times divided over the batch.
    static constexpr int kBatch = 16;

    void work(Shard* c, bool to_gpu) {
        pin_self(c->core);
        Stage01& st = *c->st;
        const std::size_t cap = c->samples.size();
        Msg m[kBatch];
        int x[kBatch], y[kBatch], x1[kBatch], y1[kBatch], k1[kBatch];
        std::uint8_t full0[kBatch], full1[kBatch], pass0[kBatch], pass1[kBatch];
        alignas(32) float f0[kBatch * 2], s0[kBatch * 12], in1[kBatch * 12], s1[kBatch * 24];
        auto seg = [&](int s, std::uint64_t a, std::uint64_t b, int n) {
            c->seg_ns[s].fetch_add(b - a, std::memory_order_relaxed);
            c->seg_n[s].fetch_add((std::uint64_t)n, std::memory_order_relaxed);
        };
        bool eof = false;
        while (!eof) {
            int n = 0;
            while (n < kBatch && c->q->try_pop(m[n])) {
                if (m[n].eof) {
                    eof = true;
                    break;
                }
                ++n;
            }
            if (n == 0) {
                if (!eof) cpu_relax();
                continue;
            }
            const std::uint64_t a = mono_ns();
            for (int i = 0; i < n; ++i) {
                x[i] = (int)m[i].x;
                y[i] = (int)m[i].y;
                st.preprocess(m[i].t, x[i], y[i], m[i].p, f0 + 2 * i);
            }
            const std::uint64_t b = mono_ns();
            seg(SEG_PRE, a, b, n);
            int n1 = 0, n_own = 0;
            if (to_gpu) {
                // tdrop first: stage outputs nobody consumes run state-only
                for (int i = 0; i < n; ++i) {
                    pass0[i] = pass1[i] = 0;
                    if (m[i].owner) {
                        ++n_own;
                        pass0[i] = st.tdrop_at(0, x[i] >> 1, y[i] >> 1);
                        if (pass0[i]) {
                            pass1[i] = st.tdrop_at(1, x[i] >> 2, y[i] >> 2);
                            k1[n1] = i;
                            x1[n1] = x[i] >> 1;
                            y1[n1] = y[i] >> 1;
                            full1[n1] = pass1[i];
                            ++n1;
                        }
                    }
                    full0[i] = pass0[i];
                }
                const std::uint64_t t1 = mono_ns();
                seg(SEG_TD0, b, t1, n);
                st.stage0_batch(n, x, y, f0, full0, s0);
                const std::uint64_t t2 = mono_ns();
                seg(SEG_S0, t1, t2, n);
                if (n1) {
                    for (int j = 0; j < n1; ++j) std::memcpy(in1 + 12 * j, s0 + 12 * k1[j], sizeof(float) * 12);
                    st.stage1_batch(n1, x1, y1, in1, full1, s1);
                    const std::uint64_t t3 = mono_ns();
                    seg(SEG_S1, t2, t3, n1);
                    if (attached.load(std::memory_order_acquire)) {
                        int np = 0;
                        for (int j = 0; j < n1; ++j) {
                            if (!full1[j]) continue;
                            publish(x1[j] >> 1, y1[j] >> 1, m[k1[j]].t, s1 + 24 * j, m[k1[j]].t_emit_ns);
                            ++np;
                        }
                        if (np) seg(SEG_PUSH, t3, mono_ns(), np);
                    }
                }
            } else {
                for (int i = 0; i < n; ++i) {
                    full0[i] = m[i].owner;
                    n_own += m[i].owner;
                }
                st.stage0_batch(n, x, y, f0, full0, s0);
                const std::uint64_t t1 = mono_ns();
                seg(SEG_S0, b, t1, n);
                for (int i = 0; i < n; ++i) {
                    pass0[i] = pass1[i] = 0;
                    if (!m[i].owner) continue;
                    pass0[i] = st.tdrop_at(0, x[i] >> 1, y[i] >> 1);
                    if (pass0[i]) {
                        k1[n1] = i;
                        x1[n1] = x[i] >> 1;
                        y1[n1] = y[i] >> 1;
                        full1[n1] = 1;
                        std::memcpy(in1 + 12 * n1, s0 + 12 * i, sizeof(float) * 12);
                        ++n1;
                    }
                }
                const std::uint64_t t2 = mono_ns();
                seg(SEG_TD0, t1, t2, n);
                if (n1) {
                    st.stage1_batch(n1, x1, y1, in1, full1, s1);
                    const std::uint64_t t3 = mono_ns();
                    seg(SEG_S1, t2, t3, n1);
                    for (int j = 0; j < n1; ++j) pass1[k1[j]] = st.tdrop_at(1, x1[j] >> 1, y1[j] >> 1);
                    seg(SEG_TD1, t3, mono_ns(), n1);
                }
            }
            const std::uint64_t done = mono_ns();
            for (int i = 0; i < n; ++i) {
                if (!m[i].owner) continue;
                const std::size_t k = c->n_samples.fetch_add(1, std::memory_order_relaxed);
                c->samples[k % cap] = (double)(done - m[i].t_arr_ns);
                if (pass0[i]) c->pass0.fetch_add(1, std::memory_order_relaxed);
                if (pass1[i]) c->pass1.fetch_add(1, std::memory_order_relaxed);
            }
            c->owner.fetch_add((std::uint64_t)n_own, std::memory_order_relaxed);
            c->halo.fetch_add((std::uint64_t)(n - n_own), std::memory_order_relaxed);
        }
    }

    void snapshot(double* out, int n_slots) const {
        for (int i = 0; i < n_slots; ++i) out[i] = 0.0;
        std::uint64_t own = 0, hal = 0, p0 = 0, p1 = 0, occ = 0;
        std::vector<double> s;
        std::uint64_t sn[NSEG] = {}, sc[NSEG] = {};
        for (const auto& c : shards) {
            own += c->owner.load();
            hal += c->halo.load();
            p0 += c->pass0.load();
            p1 += c->pass1.load();
            occ += c->q->size();
            const std::size_t n = std::min(c->n_samples.load(), c->samples.size());
            s.insert(s.end(), c->samples.begin(), c->samples.begin() + n);
            for (int k = 0; k < NSEG; ++k) {
                sn[k] += c->seg_ns[k].load();
                sc[k] += c->seg_n[k].load();
            }
        }
        out[0] = (double)own;
        out[1] = (double)hal;
        out[2] = (double)p0;
        out[3] = (double)oob.load();
        out[4] = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        out[5] = (double)occ;
        if (!s.empty()) {
            std::sort(s.begin(), s.end());
            const double n = (double)s.size();
            auto pct = [&](double q) {   // linear interpolation (include/lat_stats.h:33-40)
                if (s.size() == 1) return s[0];
                const double idx = q * (n - 1);
                const std::size_t lo = (std::size_t)std::floor(idx);
                const std::size_t hi = std::min(s.size() - 1, lo + 1);
                return s[lo] * (1.0 - (idx - lo)) + s[hi] * (idx - lo);
            };
            double mean = 0.0;
            for (double v : s) mean += v;
            out[6] = pct(0.50) * 1e-3;
            out[7] = pct(0.90) * 1e-3;
            out[8] = pct(0.99) * 1e-3;
            out[9] = pct(0.999) * 1e-3;
            out[10] = s.back() * 1e-3;
            out[11] = mean / n * 1e-3;
            out[12] = n;
        }
        out[13] = (double)p1;
        if (n_slots > 14) {
            out[14] = (double)rings[0].pushed.load();
            out[15] = (double)rings[1].pushed.load();
        }
        if (n_slots >= 28) {
            for (int k = 0; k < NSEG; ++k) {
                out[16 + k] = (double)sn[k];
                out[22 + k] = (double)sc[k];
            }
        }
        if (n_slots >= 31) {
            out[28] = (double)bp_waits.load();
            out[29] = (double)bp_wait_ns.load();
            out[30] = (double)bp_overruns.load();
        }
    }

    void reset_stats() {
        for (auto& c : shards) {
            c->owner = 0;
            c->halo = 0;
            c->pass0 = 0;
            c->pass1 = 0;
            c->n_samples = 0;
            for (int k = 0; k < NSEG; ++k) {
                c->seg_ns[k] = 0;
                c->seg_n[k] = 0;
            }
        }
        for (auto& r : rings) r.pushed = 0;
        bp_waits = 0;
        bp_wait_ns = 0;
        bp_overruns = 0;
        oob = 0;
        t0 = std::chrono::steady_clock::now();
    }

    void stop_synth() {
        if (synth_on.exchange(false) && synth.joinable()) synth.join();
        if (synth.joinable()) synth.join();
    }

    void shutdown() {
        stop_synth();
        for (auto& c : shards) {
            Msg m{};
            m.eof = 1;
            c->q->push(m);
        }
        for (auto& t : threads)
            if (t.joinable()) t.join();
    }
};

namespace {

Producer* make_producer(const char* dir, int n_shards, int halo, int base_core, int sample_cap,
                        unsigned shard_cap, bool to_gpu, const char* tag) {
    if (!dir) return nullptr;
    if (n_shards < 1) n_shards = 1;
    if (sample_cap < 1024) sample_cap = 1024;
    if (shard_cap < 4) shard_cap = 4;
    unsigned p2 = 1;
    while (p2 < shard_cap) p2 <<= 1;
    auto P = std::make_unique<Producer>();
    P->N = n_shards;
    P->halo = halo;
    try {
        for (int k = 0; k < n_shards; ++k) {
            auto c = std::make_unique<Shard>();
            c->id = k;
            c->core = base_core >= 0 ? base_core + k : -1;
            c->st = std::make_unique<Stage01>(dir);
            c->q = std::make_unique<Queue<Msg>>(p2);
            c->samples.assign((std::size_t)sample_cap, 0.0);
            P->shards.push_back(std::move(c));
        }
    } catch (const std::exception& e) {
        std::fprintf(stderr, "[%s] load failed: %s\n", tag, e.what());
        return nullptr;
    }
    P->W = P->shards[0]->st->W();
    P->H = P->shards[0]->st->H();
    P->strip = (P->W + n_shards - 1) / n_shards;
    P->t0 = std::chrono::steady_clock::now();
    Producer* raw = P.release();
    try {
        for (int k = 0; k < n_shards; ++k)
            raw->threads.emplace_back([raw, k, to_gpu]() { raw->work(raw->shards[k].get(), to_gpu); });
    } catch (const std::exception& e) {
        // threads already started take their end-of-stream message and exit
        std::fprintf(stderr, "[%s] shard threads: %s\n", tag, e.what());
        raw->shutdown();
        delete raw;
        return nullptr;
    }
    return raw;
}

int submit(Producer* P, const float* ev, int n) {
    if (!P || !ev || n <= 0) return 0;
    int accepted = 0;
    for (int i = 0; i < n; ++i) {
        const float* e = ev + 4 * (size_t)i;
        const int ex = (int)e[1], ey = (int)e[2];
        if (ex < 0 || ex >= P->W || ey < 0 || ey >= P->H) {
            P->oob.fetch_add(1, std::memory_order_relaxed);
            continue;
        }
        P->route(e[0], e[1], e[2], e[3], mono_ns());
        ++accepted;
    }
    return accepted;
}

// Paced source: one event every 1 / rate, spin-waiting on the raw monotonic
// clock; event time advances 1 / rate_mev microseconds per event.
//   uniform (lib_stage01_to_gpu.cpp:624-706): xorshift64 (13, 7, 17) with
//     seed 0x9E3779B97F4A7C15 when 0; x = r mod W, y = (r >> 16) mod H,
//     p = bit 32 of r -- the same stream for the same seed;
//   blobs: n_blobs Gaussian blobs moving at 0.5-2 px/ms and reflecting off
//     the sensor edges, plus bg_frac uniform background, p = +-1.  The blob
//     centres are recomputed every 64 events (32 us at 2 Mev/s, when a blob
//     has moved at most 0.064 px) and the Gaussian offsets come in
//     Box-Muller pairs from the xorshift stream: at 2 Mev/s the loop has
//     500 ns per event, and generation, the clock and the queue pushes share
//     them.
void synth_loop(Producer* P, double rate_mev, int core, std::uint64_t seed, int n_blobs,
                double sigma, double bg_frac) {
    pin_self(core);
    const int W = P->W, H = P->H;
    const double period_ns = rate_mev > 0 ? 1e3 / rate_mev : 0.0;
    const float dt_us = rate_mev > 0 ? (float)(1.0 / rate_mev) : 1.0f;
    std::uint64_t xs = seed ? seed : 0x9E3779B97F4A7C15ull;
    auto next_u64 = [&xs]() {
        xs ^= xs << 13;
        xs ^= xs >> 7;
        xs ^= xs << 17;
        return xs;
    };
    std::mt19937_64 rng(xs);
    std::uniform_real_distribution<double> U(0.0, 1.0);
    struct Blob { double x0, y0, vx, vy; };
    std::vector<Blob> blobs((std::size_t)std::max(0, n_blobs));
    for (auto& b : blobs) {
        b.x0 = U(rng) * (W - 1);
        b.y0 = U(rng) * (H - 1);
        const double sp = (0.5 + 1.5 * U(rng)) * 1e-3;     // px per microsecond
        const double an = 2.0 * M_PI * U(rng);
        b.vx = sp * std::cos(an);
        b.vy = sp * std::sin(an);
    }
    auto reflect = [](double v, double hi) {
        const double per = 2.0 * hi;
        double m = std::fmod(v, per);
        if (m < 0) m += per;
        return m > hi ? per - m : m;
    };
    // uniform in [0, 1) and in (0, 1] from the top 53 bits of the stream
    auto u01 = [&]() { return (double)(next_u64() >> 11) * 0x1.0p-53; };
    auto u01_open = [&]() { return (double)((next_u64() >> 11) + 1) * 0x1.0p-53; };
    constexpr int kRefresh = 64;
    const std::size_t nb = blobs.size();
    std::vector<double> cx(nb), cy(nb);
    double next = (double)mono_ns();
    float t_us = 0.f;
    std::uint64_t count = 0;
    while (P->synth_on.load(std::memory_order_relaxed)) {
        std::uint64_t now = mono_ns();
        if (period_ns > 0) {
            while ((double)now < next) {
                cpu_relax();
                now = mono_ns();
            }
            next += period_ns;
        }
        t_us += dt_us;
        float x, y, p;
        if (blobs.empty()) {
            const std::uint64_t r = next_u64();
            x = (float)(int)(r % (std::uint64_t)W);
            y = (float)(int)((r >> 16) % (std::uint64_t)H);
            p = (float)((r >> 32) & 1ull);
        } else {
            if (count % kRefresh == 0)
                for (std::size_t i = 0; i < nb; ++i) {
                    cx[i] = reflect(blobs[i].x0 + blobs[i].vx * t_us, W - 1);
                    cy[i] = reflect(blobs[i].y0 + blobs[i].vy * t_us, H - 1);
                }
            double fx, fy;
            if (u01() < bg_frac) {
                fx = std::floor(u01() * W);
                fy = std::floor(u01() * H);
            } else {
                const std::size_t i = std::min(nb - 1, (std::size_t)(u01() * (double)nb));
                const double rad = std::sqrt(-2.0 * std::log(u01_open()));
                const double ang = 2.0 * M_PI * u01();
                fx = std::rint(cx[i] + sigma * rad * std::cos(ang));
                fy = std::rint(cy[i] + sigma * rad * std::sin(ang));
            }
            x = (float)std::min<double>(W - 1, std::max(0.0, fx));
            y = (float)std::min<double>(H - 1, std::max(0.0, fy));
            p = (next_u64() >> 63) ? 1.f : -1.f;
        }
        P->route(t_us, x, y, p, now, now);
        P->synth_n.store(++count, std::memory_order_relaxed);
    }
}

[[maybe_unused]] void start_synth(Producer* P, double rate, int core, std::uint64_t seed, int n_blobs, double sigma,
                 double bg) {
    if (!P || P->synth_on.load()) return;
    if (P->synth.joinable()) P->synth.join();
    P->synth_n = 0;
    P->synth_on = true;
    try {
        P->synth = std::thread(synth_loop, P, rate, core, seed, n_blobs, sigma, bg);
    } catch (const std::exception& e) {
        std::fprintf(stderr, "[s01g] synthetic source thread: %s\n", e.what());
        P->synth_on = false;
    }
}

}  // namespace
}  // namespace ssla

using ssla::Producer;

#ifdef STAGE01_TO_GPU
#include "stage01_to_gpu.h"

struct S01gHandle : Producer {};

extern "C" {

S01gHandle* s01g_init_full(const char* dir, int n_shards, int halo, int base_core, int sample_cap,
                           unsigned int shard_ring_cap) {
    return static_cast<S01gHandle*>(
        ssla::make_producer(dir, n_shards, halo, base_core, sample_cap, shard_ring_cap, true, "s01g_init"));
}

S01gHandle* s01g_init(const char* dir, int n_shards, int halo, int base_core, int sample_cap) {
    return s01g_init_full(dir, n_shards, halo, base_core, sample_cap, 1u << 16);
}

void s01g_attach_gpu_rings_multi(S01gHandle* h, int n, void* const* bufs, void* const* heads,
                                 unsigned long long mask, int W2, int H2, const int* xlo,
                                 const int* xhi, const int* ylo, const int* yhi) {
    if (!h || n <= 0 || n > ssla::kMaxRings || !bufs || !heads || !xlo || !xhi || !ylo || !yhi) return;
    h->attached.store(false, std::memory_order_release);
    for (int b = 0; b < n; ++b) {
        ssla::RingOut& r = h->rings[b];
        r.buf = static_cast<HybridInputRec*>(bufs[b]);
        r.head = static_cast<std::uint64_t*>(heads[b]);
        r.x_lo = xlo[b];
        r.x_hi = xhi[b];
        r.y_lo = ylo[b];
        r.y_hi = yhi[b];
        r.pushed = 0;
        r.tail = nullptr;
    }
    h->n_rings = n;
    h->ring_mask = mask;
    h->W2 = W2;
    h->H2 = H2;
    h->attached.store(true, std::memory_order_release);
}

void s01g_attach_gpu_rings(S01gHandle* h, void* buf0, void* head0, void* buf1, void* head1,
                           unsigned long long mask, int W2, int H2, int lo0, int hi0, int lo1,
                           int hi1) {
    void* bufs[2] = {buf0, buf1};
    void* heads[2] = {head0, head1};
    const int xlo[2] = {lo0, lo1}, xhi[2] = {hi0, hi1}, ylo[2] = {0, 0}, yhi[2] = {H2, H2};
    s01g_attach_gpu_rings_multi(h, 2, bufs, heads, mask, W2, H2, xlo, xhi, ylo, yhi);
}

void s01g_set_ring_tails(S01gHandle* h, int n, const unsigned long long* const* tails,
                         unsigned long long timeout_ns) {
    if (!h || n < 0 || n > h->n_rings) return;
    h->bp_timeout_ns = timeout_ns;
    for (int b = 0; b < h->n_rings; ++b)
        h->rings[b].tail = (tails && b < n) ? reinterpret_cast<const std::uint64_t*>(tails[b]) : nullptr;
}

int s01g_submit_batch(S01gHandle* h, const float* ev, int n) { return ssla::submit(h, ev, n); }

void s01g_snapshot_stats(S01gHandle* h, double* out) {
    if (!out) return;
    if (!h) {
        for (int i = 0; i < 32; ++i) out[i] = 0.0;
        return;
    }
    h->snapshot(out, 32);
}

void s01g_reset_stats(S01gHandle* h) {
    if (h) h->reset_stats();
}

void s01g_shutdown(S01gHandle* h) {
    if (!h) return;
    h->shutdown();
    delete h;
}

void s01g_start_synthetic(S01gHandle* h, double rate_mev, int pin_core, unsigned long long seed) {
    ssla::start_synth(h, rate_mev, pin_core, seed, 0, 0.0, 1.0);
}

void s01g_start_synthetic_blobs(S01gHandle* h, double rate_mev, int pin_core,
                                unsigned long long seed, int n_blobs, double sigma_px,
                                double bg_frac) {
    ssla::start_synth(h, rate_mev, pin_core, seed, n_blobs < 1 ? 1 : n_blobs, sigma_px, bg_frac);
}

void s01g_stop_synthetic(S01gHandle* h) {
    if (h) h->stop_synth();
}

unsigned long long s01g_synthetic_n_pushed(S01gHandle* h) {
    return h ? h->synth_n.load() : 0ull;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Replay of ring records into several rings (multi-stream live benchmark)
// ---------------------------------------------------------------------------
struct S01gReplay {
    std::vector<HybridInputRec*> bufs;
    std::vector<std::uint64_t*> heads;
    std::vector<const HybridInputRec*> recs;
    std::vector<int> counts;
    std::uint64_t mask = 0;
    double period_ns = 0.0;
    double speed = 0.0;          // > 0: timed mode, record t (us) paces publishing
    int core = -1;
    std::atomic<bool> stop{false}, done{false};
    std::atomic<std::uint64_t> published{0};
    std::thread th;

    void put(size_t b, const HybridInputRec& r) {
        const std::uint64_t slot = __atomic_fetch_add(heads[b], 1ull, __ATOMIC_RELAXED);
        HybridInputRec* d = bufs[b] + (slot & mask);
        d->t = r.t;
        d->x = r.x;
        d->y = r.y;
        std::memcpy(d->feat1, r.feat1, sizeof(float) * SSLA_C1);
        const std::uint64_t now = ssla::mono_ns();
        d->t_push_ns = now;
        d->t_emit_ns = now;
        __atomic_store_n(&d->seq_done, slot + 1ull, __ATOMIC_RELEASE);
        published.fetch_add(1, std::memory_order_relaxed);
    }

    // timed mode: all rings merged in record-time order (ties to the lower
    // ring); a record with time t is published (t - t_first) / speed us
    // after the start, so records that sit in several rings (halo copies)
    // go out together
    void run_timed() {
        ssla::pin_self(core);
        std::vector<int> cur(bufs.size(), 0);
        double t_first = 1e300;
        for (size_t b = 0; b < bufs.size(); ++b)
            if (counts[b] > 0) t_first = std::min(t_first, (double)recs[b][0].t);
        const double start = (double)ssla::mono_ns();
        while (!stop.load(std::memory_order_relaxed)) {
            int best = -1;
            double tb = 0.0;
            for (size_t b = 0; b < bufs.size(); ++b) {
                if (cur[b] >= counts[b]) continue;
                const double t = recs[b][cur[b]].t;
                if (best < 0 || t < tb) {
                    best = (int)b;
                    tb = t;
                }
            }
            if (best < 0) break;
            const double due = start + (tb - t_first) * 1e3 / speed;
            while ((double)ssla::mono_ns() < due) ssla::cpu_relax();
            put((size_t)best, recs[best][cur[best]]);
            ++cur[best];
        }
        done.store(true, std::memory_order_release);
    }

    void run() {
        if (speed > 0.0) {
            run_timed();
            return;
        }
        ssla::pin_self(core);
        int most = 0;
        for (int c : counts) most = std::max(most, c);
        double next = (double)ssla::mono_ns();
        for (int k = 0; k < most && !stop.load(std::memory_order_relaxed); ++k) {
            for (size_t b = 0; b < bufs.size(); ++b) {
                if (k >= counts[b]) continue;
                if (period_ns > 0) {
                    while ((double)ssla::mono_ns() < next) ssla::cpu_relax();
                    next += period_ns;
                }
                put(b, recs[b][k]);
            }
        }
        done.store(true, std::memory_order_release);
    }
};

extern "C" {

static S01gReplay* replay_start(int n_rings, void* const* ring_bufs, void* const* ring_heads,
                                unsigned long long ring_mask, const void* const* records,
                                const int* counts, double rate_rec_s, double speed, int pin_core);

S01gReplay* s01g_replay_start(int n_rings, void* const* ring_bufs, void* const* ring_heads,
                              unsigned long long ring_mask, const void* const* records,
                              const int* counts, double rate_rec_s, int pin_core) {
    return replay_start(n_rings, ring_bufs, ring_heads, ring_mask, records, counts, rate_rec_s, 0.0,
                        pin_core);
}

S01gReplay* s01g_replay_start_timed(int n_rings, void* const* ring_bufs, void* const* ring_heads,
                                    unsigned long long ring_mask, const void* const* records,
                                    const int* counts, double speed, int pin_core) {
    if (!(speed > 0.0)) return nullptr;
    return replay_start(n_rings, ring_bufs, ring_heads, ring_mask, records, counts, 0.0, speed,
                        pin_core);
}

static S01gReplay* replay_start(int n_rings, void* const* ring_bufs, void* const* ring_heads,
                                unsigned long long ring_mask, const void* const* records,
                                const int* counts, double rate_rec_s, double speed, int pin_core) {
    if (n_rings <= 0 || n_rings > 64 || !ring_bufs || !ring_heads || !records || !counts)
        return nullptr;
    if ((ring_mask & (ring_mask + 1)) != 0) return nullptr;
    auto* r = new S01gReplay();
    for (int b = 0; b < n_rings; ++b) {
        if (!ring_bufs[b] || !ring_heads[b] || counts[b] < 0 || (counts[b] > 0 && !records[b])) {
            delete r;
            return nullptr;
        }
        r->bufs.push_back(static_cast<HybridInputRec*>(ring_bufs[b]));
        r->heads.push_back(static_cast<std::uint64_t*>(ring_heads[b]));
        r->recs.push_back(static_cast<const HybridInputRec*>(records[b]));
        r->counts.push_back(counts[b]);
    }
    r->mask = ring_mask;
    r->period_ns = rate_rec_s > 0 ? 1e9 / rate_rec_s : 0.0;
    r->speed = speed;
    r->core = pin_core;
    try {
        r->th = std::thread([r]() { r->run(); });
    } catch (const std::exception& e) {
        std::fprintf(stderr, "[s01g] replay thread: %s\n", e.what());
        delete r;
        return nullptr;
    }
    return r;
}

int s01g_replay_done(S01gReplay* r) { return r && r->done.load(std::memory_order_acquire) ? 1 : 0; }

unsigned long long s01g_replay_published(S01gReplay* r) { return r ? r->published.load() : 0ull; }

void s01g_replay_stop(S01gReplay* r) {
    if (!r) return;
    r->stop.store(true);
    if (r->th.joinable()) r->th.join();
    delete r;
}

}  // extern "C"

#else
#include "stage01_capi.h"

struct S0Handle : Producer {};

extern "C" {

S0Handle* s0_init(const char* dir, int n_shards, int halo, int base_core, int sample_cap) {
    return static_cast<S0Handle*>(
        ssla::make_producer(dir, n_shards, halo, base_core, sample_cap, 1u << 16, false, "s0_init"));
}

int s0_submit_batch(S0Handle* h, const float* ev, int n) { return ssla::submit(h, ev, n); }

void s0_snapshot_stats(S0Handle* h, double* out) {
    if (!out) return;
    if (!h) {
        for (int i = 0; i < 16; ++i) out[i] = 0.0;
        return;
    }
    h->snapshot(out, 14);
    out[14] = out[15] = 0.0;
}

void s0_reset_stats(S0Handle* h) {
    if (h) h->reset_stats();
}

void s0_shutdown(S0Handle* h) {
    if (!h) return;
    h->shutdown();
    delete h;
}

}  // extern "C"
#endif
