// urb_oracle.cpp -- CPU restatement of the reference's routed-expert MoE path.
//
// TEST INFRASTRUCTURE ONLY (parity checker and timed CPU baseline); see urb_oracle.h.
// Every function names the reference function it restates as file:line into
// inspirewind/Urbilateria 0.2.4.  Build flags matter: -ffp-contract=off keeps every
// separate multiply/add of the reference separate, and fmaf() is written out wherever the
// reference uses _mm256_fmadd_ps.

#include "urb_oracle.h"

#include <sched.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstring>
#include <fstream>
#include <functional>
#include <mutex>
#include <set>
#include <sstream>
#include <string>
#include <thread>
#include <tuple>
#include <vector>

namespace {

// ------------------------------------------------------------------------------------------
// Bit helpers
// ------------------------------------------------------------------------------------------
inline uint32_t f2u(float v) { uint32_t u; std::memcpy(&u, &v, 4); return u; }
inline float u2f(uint32_t u) { float v; std::memcpy(&v, &u, 4); return v; }

// f32::total_cmp key (Rust core::f32::total_cmp): flip the magnitude bits of negatives and
// compare as signed integers.
inline int32_t total_key(float v) {
    int32_t b = (int32_t)f2u(v);
    b ^= (int32_t)(((uint32_t)(b >> 31)) >> 1);
    return b;
}

// src/math/mxfp.rs:53-57 decode_e8m0_unchecked: the biased exponent field; code 0 is 2^-127.
inline float e8m0(uint8_t code) {
    uint32_t bits = (uint32_t)code << 23;
    return u2f(bits == 0 ? 0x00400000u : bits);
}

// src/math/mxfp.rs:73-79 E2M1_TABLE / decode_e2m1 (code 8 decodes to +0.0).
const float kE2M1[16] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
                         0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

// src/math/mxfp.rs:59-71 decode_e4m3fn.
float e4m3_decode(uint8_t value) {
    float sign = (value & 0x80) == 0 ? 1.0f : -1.0f;
    int exponent = (value >> 3) & 0x0f;
    int mantissa = value & 0x07;
    if (exponent == 0) return sign * (float)mantissa * std::ldexp(1.0f, -9);
    if (exponent == 0x0f && mantissa == 0x07) return NAN;
    return sign * (1.0f + (float)mantissa / 8.0f) * std::ldexp(1.0f, exponent - 7);
}

struct E4m3Table {
    float v[256];
    E4m3Table() { for (int c = 0; c < 256; ++c) v[c] = e4m3_decode((uint8_t)c); }
};
const E4m3Table &e4m3_table() { static const E4m3Table t; return t; }

// src/model/bf16.rs:478-482 decode_bf16 (little-endian u16 -> high half of an f32).
inline float bf16_at(const uint8_t *row, size_t col) {
    uint32_t bits = (uint32_t)row[2 * col] | ((uint32_t)row[2 * col + 1] << 8);
    return u2f(bits << 16);
}

// src/models/qwen3_8/math.rs:66-78 round_to_bf16 (RNE; errors on non-finite input/output).
inline bool rne_bf16(float value, float *out) {
    if (!std::isfinite(value)) return false;
    uint32_t bits = f2u(value);
    uint32_t bias = 0x7fffu + ((bits >> 16) & 1u);
    float rounded = u2f((bits + bias) & 0xffff0000u);
    if (!std::isfinite(rounded)) return false;
    *out = rounded;
    return true;
}

// ------------------------------------------------------------------------------------------
// Row-parallel pool: src/execution.rs:19, 154-160 (PARALLEL_MIN_WORK = 64 Ki MACs, one
// persistent pool).  Each task computes whole rows, so results do not depend on the width.
// ------------------------------------------------------------------------------------------
constexpr size_t kParallelMinWork = 64 * 1024;

// ------------------------------------------------------------------------------------------
// CPU topology and pinning: src/execution.rs:254-394.  The logical CPUs of the allowed set
// (/proc/self/status Cpus_allowed_list) with their (package, core) ids from sysfs, ordered so
// every physical core gets one CPU before any SMT sibling (physical_core_first); the default
// pool width is the number of physical cores (recommended_worker_threads), and worker i is
// pinned to the i-th CPU of that order (the pool's start_handler).
// ------------------------------------------------------------------------------------------
bool parse_cpu_list(const std::string &value, std::vector<int> *out) {
    std::stringstream ss(value);
    std::string part;
    while (std::getline(ss, part, ',')) {
        const size_t dash = part.find('-');
        try {
            const int a = std::stoi(part.substr(0, dash));
            const int b = dash == std::string::npos ? a : std::stoi(part.substr(dash + 1));
            if (b < a) return false;
            for (int c = a; c <= b; ++c) out->push_back(c);
        } catch (...) {
            return false;
        }
    }
    return true;
}

// (cpu, package, core) of the allowed logical CPUs, sorted by cpu (available_cpu_topology).
std::vector<std::tuple<int, int, int>> cpu_topology() {
    std::set<int> allowed;
    bool have_allowed = false;
    std::ifstream status("/proc/self/status");
    for (std::string line; std::getline(status, line);) {
        const std::string key = "Cpus_allowed_list:";
        if (line.compare(0, key.size(), key) == 0) {
            std::vector<int> cpus;
            std::string v = line.substr(key.size());
            v.erase(0, v.find_first_not_of(" \t"));
            if (parse_cpu_list(v, &cpus)) {
                allowed.insert(cpus.begin(), cpus.end());
                have_allowed = true;
            }
        }
    }
    std::vector<std::tuple<int, int, int>> topo;
    for (int cpu = 0; cpu < 4096; ++cpu) {
        const std::string base = "/sys/devices/system/cpu/cpu" + std::to_string(cpu) + "/topology/";
        std::ifstream pk(base + "physical_package_id"), co(base + "core_id");
        int package, core;
        if (!(pk >> package) || !(co >> core)) continue;
        if (have_allowed && !allowed.count(cpu)) continue;
        topo.emplace_back(cpu, package, core);
    }
    return topo;
}

std::vector<int> physical_core_first_order() {
    std::set<std::pair<int, int>> seen;
    std::vector<int> primary, siblings;
    for (const auto &t : cpu_topology()) {
        if (seen.insert({std::get<1>(t), std::get<2>(t)}).second)
            primary.push_back(std::get<0>(t));
        else
            siblings.push_back(std::get<0>(t));
    }
    primary.insert(primary.end(), siblings.begin(), siblings.end());
    return primary;
}

int physical_core_count() {
    std::set<std::pair<int, int>> cores;
    for (const auto &t : cpu_topology()) cores.insert({std::get<1>(t), std::get<2>(t)});
    return (int)cores.size();
}

void pin_current_thread(int cpu) {  // best effort, as the reference
    if (cpu < 0 || cpu >= CPU_SETSIZE) return;
    cpu_set_t set;
    CPU_ZERO(&set);
    CPU_SET(cpu, &set);
    (void)sched_setaffinity(0, sizeof(set), &set);
}

std::atomic<int> g_pin_workers{0};

// The pool: n worker threads run every parallel loop while the caller waits, as calls entering
// the reference's Rayon pool (install) do.  With pinning on, worker i runs on the i-th CPU of
// the physical-core-first order.
class Pool {
  public:
    Pool(int n, bool pin) : n_(n), pin_(pin) {
        const std::vector<int> order = pin ? physical_core_first_order() : std::vector<int>();
        for (int i = 0; i < n_ && n_ > 1; ++i) {
            const int cpu = i < (int)order.size() ? order[i] : -1;
            workers_.emplace_back([this, cpu] {
                if (cpu >= 0) pin_current_thread(cpu);
                loop();
            });
        }
    }
    ~Pool() {
        { std::lock_guard<std::mutex> g(m_); stop_ = true; }
        cv_.notify_all();
        for (auto &t : workers_) t.join();
    }
    int size() const { return n_; }
    bool pinned() const { return pin_; }
    void run(size_t items, const std::function<void(size_t)> &fn) {
        if (n_ <= 1 || items <= 1) {
            for (size_t i = 0; i < items; ++i) fn(i);
            return;
        }
        std::unique_lock<std::mutex> g(m_);
        fn_ = &fn;
        items_ = items;
        next_.store(0);
        active_ = (int)workers_.size();
        ++generation_;
        cv_.notify_all();
        done_cv_.wait(g, [this] { return active_ == 0; });
        fn_ = nullptr;
    }

  private:
    void drain() {
        for (;;) {
            size_t i = next_.fetch_add(1);
            if (i >= items_) break;
            (*fn_)(i);
        }
    }
    void loop() {
        uint64_t seen = 0;
        for (;;) {
            {
                std::unique_lock<std::mutex> g(m_);
                cv_.wait(g, [&] { return stop_ || generation_ != seen; });
                if (stop_) return;
                seen = generation_;
            }
            drain();
            {
                std::lock_guard<std::mutex> g(m_);
                if (--active_ == 0) done_cv_.notify_all();
            }
        }
    }
    int n_;
    bool pin_;
    std::vector<std::thread> workers_;
    std::mutex m_;
    std::condition_variable cv_, done_cv_;
    const std::function<void(size_t)> *fn_ = nullptr;
    size_t items_ = 0;
    std::atomic<size_t> next_{0};
    int active_ = 0;
    uint64_t generation_ = 0;
    bool stop_ = false;
};

std::mutex g_pool_mutex;
Pool *g_pool = nullptr;

Pool &pool(int threads) {
    std::lock_guard<std::mutex> g(g_pool_mutex);
    if (threads < 1) threads = 1;
    const bool pin = g_pin_workers.load() != 0;
    if (!g_pool || g_pool->size() != threads || g_pool->pinned() != pin) {
        delete g_pool;
        g_pool = new Pool(threads, pin);
    }
    return *g_pool;
}

// Runs fn(row_begin, row_end) over [0, rows) in row chunks.  Serial when the reference
// would not parallelise (src/execution.rs:154-156).
void for_rows(Pool &p, size_t rows, size_t work,
              const std::function<void(size_t, size_t)> &fn) {
    if (p.size() <= 1 || rows <= 1 || work < kParallelMinWork) {
        fn(0, rows);
        return;
    }
    size_t chunk = std::max<size_t>(1, rows / (size_t)(p.size() * 8));
    size_t items = (rows + chunk - 1) / chunk;
    p.run(items, [&](size_t i) {
        size_t b = i * chunk, e = std::min(rows, b + chunk);
        fn(b, e);
    });
}

bool all_finite(const float *v, size_t n) {
    for (size_t i = 0; i < n; ++i)
        if (!std::isfinite(v[i])) return false;
    return true;
}

// ------------------------------------------------------------------------------------------
// Per-row dot products.  `x` holds `batch` token rows of `cols` floats; `out[b]` receives the
// dot of this weight row with token b.  Every token keeps the single-token reduction order
// (the reference's batch kernels are tested bit-identical to independent matvecs:
// src/model/bf16.rs:860-887, src/math/mxfp.rs:2347-2383, 2595-2628).
// ------------------------------------------------------------------------------------------

// src/model/bf16.rs:484-500 dot_bf16 / :492-534 dot_bf16_f64_ordered_avx2:
// ordered f64 additions starting from -0.0 (Iterator::sum identity).
void dot_bf16_f64(const uint8_t *row, size_t cols, const float *x, size_t batch, float *out) {
    std::vector<double> sum(batch, -0.0);
    for (size_t c = 0; c < cols; ++c) {
        double w = (double)bf16_at(row, c);
        for (size_t b = 0; b < batch; ++b) sum[b] += w * (double)x[b * cols + c];
    }
    for (size_t b = 0; b < batch; ++b) out[b] = (float)sum[b];
}

// src/model/matrix.rs:236-259 Matrix::matvec_rows (F32 weights): ordered f64 additions of
// f64(w) * f64(x) from -0.0, rounded to f32 once.
void dot_f32_f64(const uint8_t *row, size_t cols, const float *x, size_t batch, float *out) {
    std::vector<double> sum(batch, -0.0);
    for (size_t c = 0; c < cols; ++c) {
        float wf;
        std::memcpy(&wf, row + 4 * c, 4);
        const double w = (double)wf;
        for (size_t b = 0; b < batch; ++b) sum[b] += w * (double)x[b * cols + c];
    }
    for (size_t b = 0; b < batch; ++b) out[b] = (float)sum[b];
}

// src/model/bf16.rs:589-610 dot_bf16_fp32_avx2_fma (also :693-741 four-row and :612-687
// batched forms, which keep this tree): lane j FMA-accumulates columns == j (mod 8) over the
// complete 8-column prefix from +0.0; lanes are summed 0..7 in order; the tail is added with a
// separate multiply and add.
void dot_bf16_fp32(const uint8_t *row, size_t cols, const float *x, size_t batch, float *out) {
    size_t complete = cols / 8 * 8;
    for (size_t b = 0; b < batch; ++b) {
        const float *xb = x + b * cols;
        float lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (size_t c = 0; c < complete; c += 8)
            for (int j = 0; j < 8; ++j) lane[j] = std::fma(bf16_at(row, c + j), xb[c + j], lane[j]);
        float sum = -0.0f;
        for (int j = 0; j < 8; ++j) sum += lane[j];
        for (size_t c = complete; c < cols; ++c) {
            float p = bf16_at(row, c) * xb[c];
            sum += p;
        }
        out[b] = sum;
    }
}

inline uint8_t nibble(const uint8_t *packed, size_t col) {
    uint8_t byte = packed[col / 2];
    return (col % 2 == 0) ? (byte & 15) : (byte >> 4);
}

// src/math/mxfp.rs:1849-1873 dot_e2m1_e8m0_f64_ordered (AVX2 form :1900-1971 is bit-equal):
// weight = decode_e2m1(code) * scale in f32, then f64 product, ordered f64 adds from +0.0.
void dot_mxfp4_f64(const uint8_t *packed, const uint8_t *scales, size_t cols, const float *x,
                   size_t batch, float *out) {
    const size_t group = 32;
    std::vector<double> sum(batch, 0.0);
    for (size_t c = 0; c < cols; ++c) {
        float w = kE2M1[nibble(packed, c)] * e8m0(scales[c / group]);
        double wd = (double)w;
        for (size_t b = 0; b < batch; ++b) sum[b] += wd * (double)x[b * cols + c];
    }
    for (size_t b = 0; b < batch; ++b) out[b] = (float)sum[b];
}

// src/math/mxfp.rs:1875-1898 dot_e2m1_e8m0_fp32_ordered: sum += (e2m1 * scale) * x in f32.
float dot_mxfp4_fp32(const uint8_t *packed, const uint8_t *scales, size_t cols, const float *x) {
    const size_t group = 32;
    float sum = 0.0f;
    for (size_t c = 0; c < cols; ++c) {
        float w = kE2M1[nibble(packed, c)] * e8m0(scales[c / group]);
        float p = w * x[c];
        sum += p;
    }
    return sum;
}

// src/math/mxfp.rs:1069-1125 dot_e4m3_e8m0_avx2_fma and :1127-1158 the aligned form
// (1x32 E8M0 blocks on AVX2+FMA hosts): w = e4m3 * scale (f32); within each 32-column block,
// 8-column groups feed 8 FMA lanes (lane j takes column == j mod 8 of the group); a partial
// block's incomplete 8-column tail goes to a scalar multiply-add accumulator; the result is
// (lane0 + ... + lane7) + scalar_tail.
void dot_mxfp8_compact(const uint8_t *codes, const uint8_t *scales, size_t cols, const float *x,
                       size_t batch, float *out) {
    const float *tab = e4m3_table().v;
    for (size_t b = 0; b < batch; ++b) {
        const float *xb = x + b * cols;
        float lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        float tail = 0.0f;
        for (size_t start = 0, blk = 0; start < cols; start += 32, ++blk) {
            size_t len = std::min<size_t>(32, cols - start);
            float scale = e8m0(scales[blk]);
            size_t complete = len / 8 * 8;
            for (size_t off = 0; off < complete; off += 8)
                for (int j = 0; j < 8; ++j) {
                    float w = tab[codes[start + off + j]] * scale;
                    lane[j] = std::fma(w, xb[start + off + j], lane[j]);
                }
            for (size_t off = complete; off < len; ++off) {
                float w = tab[codes[start + off]] * scale;
                float p = w * xb[start + off];
                tail += p;
            }
        }
        float sum = -0.0f;
        for (int j = 0; j < 8; ++j) sum += lane[j];
        out[b] = (cols % 32 == 0) ? sum : sum + tail;
    }
}

// src/math/mxfp.rs:754-765 (scalar) and :960-1013 dot_e4m3_e8m0_f64_ordered_avx2: ordered f64.
void dot_mxfp8_f64(const uint8_t *codes, const uint8_t *scales, size_t cols, const float *x,
                   size_t batch, float *out) {
    const float *tab = e4m3_table().v;
    std::vector<double> sum(batch, 0.0);
    for (size_t c = 0; c < cols; ++c) {
        double w = (double)(tab[codes[c]] * e8m0(scales[c / 32]));
        for (size_t b = 0; b < batch; ++b) sum[b] += w * (double)x[b * cols + c];
    }
    for (size_t b = 0; b < batch; ++b) out[b] = (float)sum[b];
}

size_t row_bytes(int format, size_t cols) {
    switch (format) {
    case URBO_FMT_BF16: return cols * 2;
    case URBO_FMT_MXFP4: return (cols + 1) / 2;
    case URBO_FMT_F32: return cols * 4;
    default: return cols;
    }
}

// One WeightMatrix::matvec / matmul_rows over `batch` tokens, row-parallel.
// BF16 and MXFP4: ordered f64 (src/model/weight.rs:92-101 -> bf16.rs:121-216,
// mxfp.rs:1725-1780); MXFP8 1x32: compact FMA with a non-finite output check
// (mxfp.rs:693-783).  Output layout is token-major [batch, rows].
// MxFp8Matrix::matvec_rows picks its kernel by host CPU (src/math/mxfp.rs:720-765): the compact
// 8-lane FMA kernel on AVX2+FMA hosts (the default here), ordered f64 elsewhere.
int g_mxfp8_fma_host = 1;

int weight_matmul(Pool &p, int format, const uint8_t *data, const uint8_t *scales, size_t rows,
                  size_t cols, const float *x, size_t batch, float *out) {
    if (!all_finite(x, batch * cols)) return URBO_NONFINITE;
    size_t rb = row_bytes(format, cols), sb = (cols + 31) / 32;
    for_rows(p, rows, rows * cols * batch, [&](size_t r0, size_t r1) {
        std::vector<float> tmp(batch);
        for (size_t r = r0; r < r1; ++r) {
            const uint8_t *row = data + r * rb;
            if (format == URBO_FMT_BF16) dot_bf16_f64(row, cols, x, batch, tmp.data());
            else if (format == URBO_FMT_F32) dot_f32_f64(row, cols, x, batch, tmp.data());
            else if (format == URBO_FMT_MXFP4)
                dot_mxfp4_f64(row, scales + r * sb, cols, x, batch, tmp.data());
            else if (g_mxfp8_fma_host)
                dot_mxfp8_compact(row, scales + r * sb, cols, x, batch, tmp.data());
            else dot_mxfp8_f64(row, scales + r * sb, cols, x, batch, tmp.data());
            for (size_t b = 0; b < batch; ++b) out[b * rows + r] = tmp[b];
        }
    });
    if (format == URBO_FMT_MXFP8 && !all_finite(out, batch * rows)) return URBO_NONFINITE;
    return URBO_OK;
}

// Bf16Matrix::matmul_rows_fp32 (src/model/bf16.rs:290-416; single token :223-286): the
// 8-lane FMA tree per token, non-finite outputs rejected.
int bf16_matmul_fp32(Pool &p, const uint8_t *data, size_t rows, size_t cols, const float *x,
                     size_t batch, float *out) {
    if (!all_finite(x, batch * cols)) return URBO_NONFINITE;
    for_rows(p, rows, rows * cols * batch, [&](size_t r0, size_t r1) {
        std::vector<float> tmp(batch);
        for (size_t r = r0; r < r1; ++r) {
            dot_bf16_fp32(data + r * cols * 2, cols, x, batch, tmp.data());
            for (size_t b = 0; b < batch; ++b) out[b * rows + r] = tmp[b];
        }
    });
    if (!all_finite(out, batch * rows)) return URBO_NONFINITE;
    return URBO_OK;
}

// src/models/qwen3_8/math.rs:10-55 linear / linear_batch for BF16 weights: FP32 GEMV, then
// round_to_bf16_in_place (which rejects non-finite values).
int qwen_linear(Pool &p, const uint8_t *data, size_t rows, size_t cols, const float *x,
                size_t batch, float *out) {
    int st = bf16_matmul_fp32(p, data, rows, cols, x, batch, out);
    if (st) return st;
    return urbo_round_to_bf16_in_place(out, batch * rows);
}

// WeightMatrix::matvec_fp32_accum / matmul_rows_fp32_accum (src/model/weight.rs:213-260):
// BF16 -> the 8-lane FP32 tree (bf16.rs:223-416), MXFP4 -> matvec_rows_fp32, the sequential
// f32 dot without FMA (mxfp.rs:1660-1723), other formats -> matvec.  Per-token results are
// identical to the batched kernels (mxfp.rs:2632-2665, bf16.rs:860-887).
int weight_matmul_fp32_accum(Pool &p, int format, const uint8_t *data, const uint8_t *scales,
                             size_t rows, size_t cols, const float *x, size_t batch, float *out) {
    if (format == URBO_FMT_BF16) return bf16_matmul_fp32(p, data, rows, cols, x, batch, out);
    if (format != URBO_FMT_MXFP4) return weight_matmul(p, format, data, scales, rows, cols, x,
                                                      batch, out);
    if (!all_finite(x, batch * cols)) return URBO_NONFINITE;
    const size_t rb = (cols + 1) / 2, sb = (cols + 31) / 32;
    for_rows(p, rows, rows * cols * batch, [&](size_t r0, size_t r1) {
        for (size_t r = r0; r < r1; ++r)
            for (size_t b = 0; b < batch; ++b)
                out[b * rows + r] = dot_mxfp4_fp32(data + r * rb, scales + r * sb, cols,
                                                   x + b * cols);
    });
    if (!all_finite(out, batch * rows)) return URBO_NONFINITE;
    return URBO_OK;
}

// ------------------------------------------------------------------------------------------
// Routers
// ------------------------------------------------------------------------------------------
float silu_f(float v) { return v / (1.0f + ::expf(-v)); }  // src/math/ops.rs:36-38

}  // namespace

// ==========================================================================================
// Exported element functions
// ==========================================================================================
extern "C" {

// src/math/mxfp.rs:43-50 decode_e8m0.
int urbo_decode_e8m0(uint8_t code, float *out) {
    if (code == 0xff) return URBO_INVALID_SCALE;
    *out = e8m0(code);
    return URBO_OK;
}

float urbo_decode_e2m1(uint8_t code) { return kE2M1[code & 0x0f]; }
float urbo_decode_e4m3fn(uint8_t code) { return e4m3_decode(code); }

// src/math/mxfp.rs:246-275 encode_e4m3fn_finite.
uint8_t urbo_encode_e4m3fn_finite(float value) {
    value = std::min(std::max(value, -448.0f), 448.0f);
    float magnitude = std::fabs(value);
    if (magnitude == 0.0f) return 0;
    uint32_t code;
    if (magnitude < std::ldexp(1.0f, -6)) {
        code = (uint32_t)std::nearbyint(magnitude * 512.0f);
    } else {
        const uint32_t discard = 20, round_bias = (1u << (discard - 1)) - 1;
        uint32_t bits = f2u(magnitude);
        uint32_t retained_lsb = (bits >> discard) & 1u;
        uint32_t rounded = (bits + round_bias + retained_lsb) & ~((1u << discard) - 1);
        uint32_t exponent = (rounded >> 23) & 0xffu;
        exponent = exponent > 120 ? exponent - 120 : 0;
        uint32_t mantissa = (rounded >> discard) & 0x07u;
        code = std::min<uint32_t>((exponent << 3) | mantissa, 0x7e);
    }
    if (std::signbit(value) && code != 0) code |= 0x80;
    return (uint8_t)code;
}

// src/math/mxfp.rs:300-319 power_of_two_ceiling (keeps the log2f/powf formula near powers).
float urbo_power_of_two_ceiling(float value) {
    uint32_t bits = f2u(value);
    uint32_t exponent = bits & 0x7f800000u, mantissa = bits & 0x007fffffu;
    if (mantissa == 0) return value;
    const uint32_t boundary = 4096;
    if (exponent == 0 || mantissa <= boundary || mantissa >= 0x007fffffu - boundary)
        return ::powf(2.0f, std::ceil(::log2f(value)));
    uint32_t e = exponent + 0x00800000u;
    if (e < exponent) e = 0xffffffffu;  // saturating_add
    return u2f(e);
}

// src/math/mxfp.rs:89-115 simulate_e4m3_activation_in_place.
int urbo_simulate_e4m3_activation(float *values, size_t n, size_t block) {
    if (n == 0 || block == 0) return URBO_SHAPE;
    if (!all_finite(values, n)) return URBO_NONFINITE;
    const float *tab = e4m3_table().v;
    for (size_t start = 0; start < n; start += block) {
        size_t end = std::min(n, start + block);
        float amax = 1.0e-4f;
        for (size_t i = start; i < end; ++i) amax = std::fmax(amax, std::fabs(values[i]));
        float scale = urbo_power_of_two_ceiling(amax / 448.0f);
        for (size_t i = start; i < end; ++i) {
            uint8_t code = urbo_encode_e4m3fn_finite(values[i] / scale);
            values[i] = tab[code] * scale;
        }
    }
    return URBO_OK;
}

int urbo_round_to_bf16(float value, float *out) {
    return rne_bf16(value, out) ? URBO_OK : URBO_NONFINITE;
}

// src/models/qwen3_8/math.rs:80-95: values before the first failing element are rounded, the
// failing element and everything after it are left untouched.
int urbo_round_to_bf16_in_place(float *values, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        float r;
        if (!rne_bf16(values[i], &r)) return URBO_NONFINITE;
        values[i] = r;
    }
    return URBO_OK;
}

size_t urbo_matrix_bytes(int format, size_t rows, size_t cols, size_t *scale_bytes) {
    if (scale_bytes)
        *scale_bytes = format == URBO_FMT_BF16 || format == URBO_FMT_F32 ? 0
                                                                         : rows * ((cols + 31) / 32);
    return rows * row_bytes(format, cols);
}

// Payload validation done at construction:
//   BF16  src/model/bf16.rs:62-64 (any non-finite element -> MatrixError::NonFinite)
//   MXFP4 src/math/mxfp.rs:1431-1435 (any E8M0 0xFF -> InvalidScale)
//   MXFP8 src/math/mxfp.rs:448-453 (E4M3 NaN codes first -> NonFinite, then E8M0 0xFF)
int urbo_validate(int format, const uint8_t *data, const uint8_t *scales, size_t rows,
                  size_t cols) {
    if (rows == 0 || cols == 0) return URBO_SHAPE;
    size_t sb = 0, nb = urbo_matrix_bytes(format, rows, cols, &sb);
    if (format == URBO_FMT_F32) {  // DenseMatrix::new (src/model/matrix.rs:45-63): finite data
        for (size_t i = 0; i < nb; i += 4) {
            float v;
            std::memcpy(&v, data + i, 4);
            if (!std::isfinite(v)) return URBO_NONFINITE;
        }
        return URBO_OK;
    }
    if (format == URBO_FMT_BF16) {
        for (size_t i = 0; i < nb; i += 2)
            if ((data[i + 1] & 0x7f) == 0x7f && (data[i] & 0x80)) return URBO_NONFINITE;
        return URBO_OK;
    }
    if (format == URBO_FMT_MXFP8)
        for (size_t i = 0; i < nb; ++i)
            if ((data[i] & 0x7f) == 0x7f) return URBO_NONFINITE;
    for (size_t i = 0; i < sb; ++i)
        if (scales[i] == 0xff) return URBO_INVALID_SCALE;
    return URBO_OK;
}

// Dequantised row: Bf16Matrix::write_row (bf16.rs:92-113), MxFp4Matrix::row
// (mxfp.rs:1828-1846), MxFp8Matrix::row (mxfp.rs:855-877).
int urbo_row(int format, const uint8_t *data, const uint8_t *scales, size_t rows, size_t cols,
             size_t row, float *out) {
    if (row >= rows) return URBO_SHAPE;
    size_t rb = row_bytes(format, cols), sb = (cols + 31) / 32;
    const uint8_t *r = data + row * rb;
    for (size_t c = 0; c < cols; ++c) {
        if (format == URBO_FMT_BF16) out[c] = bf16_at(r, c);
        else if (format == URBO_FMT_F32) std::memcpy(&out[c], r + 4 * c, 4);
        else if (format == URBO_FMT_MXFP4) out[c] = kE2M1[nibble(r, c)] * e8m0(scales[row * sb + c / 32]);
        else out[c] = e4m3_table().v[r[c]] * e8m0(scales[row * sb + c / 32]);
    }
    return URBO_OK;
}

int urbo_matvec_rows(int format, const uint8_t *data, const uint8_t *scales, size_t rows,
                     size_t cols, size_t start, size_t count, const float *x, float *out) {
    if (start + count > rows) return URBO_SHAPE;
    size_t rb = row_bytes(format, cols), sb = (cols + 31) / 32;
    return weight_matmul(pool(1), format, data + start * rb,
                         scales ? scales + start * sb : nullptr, count, cols, x, 1, out);
}

int urbo_bf16_matvec_rows_fp32(const uint16_t *data, size_t rows, size_t cols, size_t start,
                               size_t count, const float *x, float *out) {
    if (start + count > rows) return URBO_SHAPE;
    return bf16_matmul_fp32(pool(1), (const uint8_t *)(data + start * cols), count, cols, x, 1,
                            out);
}

// src/math/mxfp.rs:1665-1723 matvec_rows_fp32 (non-finite output -> NonFinite).
int urbo_mxfp4_matvec_rows_fp32(const uint8_t *packed, const uint8_t *scales, size_t rows,
                                size_t cols, size_t start, size_t count, const float *x,
                                float *out) {
    if (start + count > rows) return URBO_SHAPE;
    if (!all_finite(x, cols)) return URBO_NONFINITE;
    size_t rb = (cols + 1) / 2, sb = (cols + 31) / 32;
    for (size_t r = 0; r < count; ++r)
        out[r] = dot_mxfp4_fp32(packed + (start + r) * rb, scales + (start + r) * sb, cols, x);
    if (!all_finite(out, count)) return URBO_NONFINITE;
    return URBO_OK;
}

int urbo_mxfp8_matvec_rows_f64(const uint8_t *codes, const uint8_t *scales, size_t rows,
                               size_t cols, size_t start, size_t count, const float *x,
                               float *out) {
    if (start + count > rows) return URBO_SHAPE;
    if (!all_finite(x, cols)) return URBO_NONFINITE;
    size_t sb = (cols + 31) / 32;
    for (size_t r = 0; r < count; ++r)
        dot_mxfp8_f64(codes + (start + r) * cols, scales + (start + r) * sb, cols, x, 1, out + r);
    if (!all_finite(out, count)) return URBO_NONFINITE;
    return URBO_OK;
}

// src/models/qwen3_8/moe.rs:91-159 route_softmax_top_k.
int urbo_route_softmax_top_k(const float *logits, size_t n, size_t top_k, int32_t *ids,
                             float *weights) {
    if (n == 0) return URBO_INVALID_GEOMETRY;
    if (top_k == 0 || top_k > n) return URBO_INVALID_GEOMETRY;
    if (!all_finite(logits, n)) return URBO_NONFINITE;
    float maximum = -INFINITY;
    for (size_t i = 0; i < n; ++i) maximum = std::fmax(maximum, logits[i]);
    std::vector<float> prob(n);
    float denominator = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        prob[i] = ::expf(logits[i] - maximum);
        denominator += prob[i];
    }
    if (!std::isfinite(denominator) || denominator <= 0.0f) return URBO_NONFINITE;
    for (size_t i = 0; i < n; ++i) prob[i] /= denominator;
    if (!all_finite(prob.data(), n)) return URBO_NONFINITE;
    std::vector<size_t> ranking(n);
    for (size_t i = 0; i < n; ++i) ranking[i] = i;
    std::stable_sort(ranking.begin(), ranking.end(), [&](size_t l, size_t r) {
        int32_t kl = total_key(prob[l]), kr = total_key(prob[r]);
        if (kl != kr) return kl > kr;
        return l < r;
    });
    ranking.resize(top_k);
    float selected = 0.0f;
    for (size_t e : ranking) selected += prob[e];
    if (!std::isfinite(selected) || selected <= 0.0f) return URBO_NONFINITE;
    for (size_t j = 0; j < top_k; ++j) {
        float w = prob[ranking[j]] / selected;
        if (!std::isfinite(w)) return URBO_NONFINITE;
        ids[j] = (int32_t)ranking[j];
        weights[j] = w;
    }
    return URBO_OK;
}

// src/math/routing.rs:38-155 route_noaux_tc.
int urbo_route_noaux_tc(const float *logits, const float *bias, size_t n, size_t top_k,
                        size_t n_group, size_t topk_group, int normalize, float scale,
                        int32_t *ids, float *weights, float *selection_out) {
    if (n == 0) return URBO_INVALID_GEOMETRY;
    std::vector<float> zero;
    if (!bias) { zero.assign(n, 0.0f); bias = zero.data(); }
    if (!all_finite(logits, n) || !all_finite(bias, n) || !std::isfinite(scale))
        return URBO_NONFINITE;
    if (scale <= 0.0f) return URBO_INVALID_GEOMETRY;
    if (n_group == 0 || n % n_group != 0) return URBO_INVALID_GEOMETRY;
    if (top_k == 0 || top_k > n) return URBO_INVALID_GEOMETRY;
    if (topk_group == 0 || topk_group > n_group) return URBO_INVALID_GEOMETRY;
    size_t per_group = n / n_group;
    if (per_group < 2) return URBO_INVALID_GEOMETRY;

    std::vector<float> gates(n), sel(n);
    for (size_t i = 0; i < n; ++i) {
        gates[i] = 1.0f / (1.0f + ::expf(-logits[i]));
        sel[i] = gates[i] + bias[i];
    }
    std::vector<std::pair<size_t, float>> groups;
    for (size_t g = 0; g < n_group; ++g) {
        std::vector<float> s(sel.begin() + g * per_group, sel.begin() + (g + 1) * per_group);
        std::stable_sort(s.begin(), s.end(),
                         [](float a, float b) { return total_key(a) > total_key(b); });
        groups.push_back({g, s[0] + s[1]});
    }
    std::stable_sort(groups.begin(), groups.end(), [](const auto &a, const auto &b) {
        int32_t ka = total_key(a.second), kb = total_key(b.second);
        if (ka != kb) return ka > kb;
        return a.first < b.first;
    });
    std::vector<char> allowed(n, 0);
    for (size_t i = 0; i < topk_group; ++i)
        std::fill(allowed.begin() + groups[i].first * per_group,
                  allowed.begin() + (groups[i].first + 1) * per_group, 1);
    std::vector<size_t> ranking;
    for (size_t i = 0; i < n; ++i)
        if (allowed[i]) ranking.push_back(i);
    std::stable_sort(ranking.begin(), ranking.end(), [&](size_t l, size_t r) {
        int32_t kl = total_key(sel[l]), kr = total_key(sel[r]);
        if (kl != kr) return kl > kr;
        return l < r;
    });
    if (ranking.size() < top_k) return URBO_INVALID_GEOMETRY;
    ranking.resize(top_k);
    float denominator = -0.0f;  // Iterator::sum identity
    for (size_t e : ranking) denominator += gates[e];
    denominator += 1e-20f;
    if (normalize && !std::isfinite(denominator)) return URBO_NONFINITE;
    for (size_t j = 0; j < top_k; ++j) {
        size_t e = ranking[j];
        float w = normalize ? gates[e] / denominator : gates[e];
        ids[j] = (int32_t)e;
        weights[j] = w * scale;
        if (selection_out) selection_out[j] = sel[e];
    }
    return URBO_OK;
}

// route_sqrt_softplus (src/models/deepseek_v4/math.rs:451-516, softplus :604-610) without hash
// experts: score = sqrt(softplus(l)); selection = score + bias ranks (desc, lower id on ties);
// weight = score / (f32 sum of the selected scores in ranking order) * scale.
static float softplus_f(float v) {
    return v > 0.0f ? v + ::log1pf(::expf(-v)) : ::log1pf(::expf(v));
}

int urbo_route_sqrt_softplus(const float *logits, const float *bias, size_t n, size_t top_k,
                             float scale, int32_t *ids, float *weights, float *selection_out) {
    return urbo_route_sqrt_softplus_hashed(logits, bias, nullptr, n, top_k, scale, ids, weights,
                                           selection_out);
}

// route_sqrt_softplus with `hash_experts` (deepseek_v4/math.rs:451-516): the checks in the
// reference's order (geometry, scale, finite logits and bias, hash ids in range), scores
// s = sqrt(softplus(l)), selection s + bias; the experts are the hash row as given (table order)
// or the top_k of the selection (value descending, lower id on ties); the denominator sums the
// chosen scores in that order from -0.0; weight = s / denominator * scale.
int urbo_route_sqrt_softplus_hashed(const float *logits, const float *bias, const int64_t *hash,
                                    size_t n, size_t top_k, float scale, int32_t *ids,
                                    float *weights, float *selection_out) {
    if (n == 0 || top_k == 0 || top_k > n) return URBO_SHAPE;
    if (!std::isfinite(scale)) return URBO_NONFINITE;
    if (scale <= 0.0f) return URBO_INVALID_GEOMETRY;  // validate_positive
    if (!all_finite(logits, n) || (bias && !all_finite(bias, n))) return URBO_NONFINITE;
    std::vector<float> score(n), sel(n);
    for (size_t i = 0; i < n; ++i) {
        score[i] = ::sqrtf(softplus_f(logits[i]));
        sel[i] = score[i] + (bias ? bias[i] : 0.0f);
    }
    std::vector<size_t> ranking;
    if (hash) {
        for (size_t j = 0; j < top_k; ++j)  // "hash expert IDs must be in range"
            if (hash[j] < 0 || (uint64_t)hash[j] >= n) return URBO_INVALID_GEOMETRY;
        for (size_t j = 0; j < top_k; ++j) ranking.push_back((size_t)hash[j]);
    } else {
        ranking.resize(n);
        for (size_t i = 0; i < n; ++i) ranking[i] = i;
        std::stable_sort(ranking.begin(), ranking.end(), [&](size_t l, size_t r) {
            int32_t kl = total_key(sel[l]), kr = total_key(sel[r]);
            if (kl != kr) return kl > kr;
            return l < r;
        });
        ranking.resize(top_k);
    }
    float denominator = -0.0f;  // Iterator::sum identity
    for (size_t e : ranking) denominator += score[e];
    if (!std::isfinite(denominator) || denominator <= 0.0f) return URBO_NONFINITE;
    for (size_t j = 0; j < top_k; ++j) {
        size_t e = ranking[j];
        ids[j] = (int32_t)e;
        weights[j] = score[e] / denominator * scale;
        if (selection_out) selection_out[j] = sel[e];
    }
    return URBO_OK;
}

float urbo_silu(float value) { return silu_f(value); }

int urbo_physical_cores(void) { return physical_core_count(); }

size_t urbo_cpu_order(int *cpus, size_t capacity) {
    const std::vector<int> order = physical_core_first_order();
    for (size_t i = 0; i < order.size() && i < capacity; ++i) cpus[i] = order[i];
    return order.size();
}

int urbo_set_pinning(int enable) { return g_pin_workers.exchange(enable ? 1 : 0); }

int urbo_set_mxfp8_fma_host(int fma_host) {
    int old = g_mxfp8_fma_host;
    g_mxfp8_fma_host = fma_host ? 1 : 0;
    return old;
}

// bounded_swiglu_in_place (src/models/deepseek_v4/math.rs:526-548): validate_positive(limit)
// (:669-677), non-finite inputs rejected, then gate' = min(gate, limit),
// up' = clamp(up, -limit, limit), out = gate' / (1 + exp(-gate')) * up'.
int urbo_bounded_swiglu(const float *gate, const float *up, size_t n, float limit, float *out) {
    if (!(std::isfinite(limit) && limit > 0.0f)) return URBO_INVALID_GEOMETRY;
    if (!all_finite(gate, n) || !all_finite(up, n)) return URBO_NONFINITE;
    for (size_t i = 0; i < n; ++i) {
        const float g = std::fmin(gate[i], limit);
        const float u = std::fmin(std::fmax(up[i], -limit), limit);
        out[i] = g / (1.0f + ::expf(-g)) * u;
    }
    return URBO_OK;
}

// ==========================================================================================
// The steps either side of the MoE call in the Qwen3.6 decoder layer.
// ==========================================================================================
// zero_centered_rms_norm (src/models/qwen3_8/norm.rs:38-52): validate (norm.rs:142-174),
// inverse_rms (norm.rs:176-186: f32 fold of value * value from 0.0, divided by the length,
// (mean_square + eps).sqrt().recip()), out = value * inverse * (1.0 + offset), finite check
// (norm.rs:188-193); then the runtime's BF16 cast (qwen3_6/runtime.rs:1053-1057).
int urbo_zc_rms_norm(const float *x, const float *weight, size_t n, size_t hidden, float eps,
                     int round_bf16, float *out) {
    if (hidden == 0) return URBO_SHAPE;
    if (!(std::isfinite(eps) && eps > 0.0f)) return URBO_INVALID_GEOMETRY;
    if (!all_finite(weight, hidden)) return URBO_NONFINITE;
    for (size_t t = 0; t < n; ++t) {
        const float *v = x + t * hidden;
        float *o = out + t * hidden;
        if (!all_finite(v, hidden)) return URBO_NONFINITE;
        float sum = 0.0f;
        for (size_t i = 0; i < hidden; ++i) sum = sum + v[i] * v[i];
        const float mean_square = sum / (float)hidden;
        const float inverse = 1.0f / std::sqrt(mean_square + eps);
        if (!std::isfinite(inverse)) return URBO_NONFINITE;
        for (size_t i = 0; i < hidden; ++i) o[i] = v[i] * inverse * (1.0f + weight[i]);
        if (!all_finite(o, hidden)) return URBO_NONFINITE;
        if (round_bf16) {
            const int st = urbo_round_to_bf16_in_place(o, hidden);
            if (st) return st;
        }
    }
    return URBO_OK;
}

// add_residual (src/models/qwen3_6/runtime.rs:1470-1494) with bf16_activations.
int urbo_add_residual_bf16(float *residual, const float *update, size_t n) {
    for (size_t i = 0; i < n; ++i) residual[i] += update[i];
    const int st = urbo_round_to_bf16_in_place(residual, n);
    if (st) return st;
    return all_finite(residual, n) ? URBO_OK : URBO_NONFINITE;
}

// ==========================================================================================
// One MoE layer.  Tokens are routed first, then grouped by expert (the reference's
// execute_batched_moe permutation, src/models/qwen3_6/runtime.rs:1123-1132: BTreeMap by
// expert id, tokens in order); each group runs the batched projections, whose per-token
// results equal the tokenwise path bit for bit; finally every token is combined in the order
// its composition prescribes.
// ==========================================================================================
namespace {

struct Group {
    size_t expert;
    std::vector<size_t> tokens;   // token ids in ascending order
    std::vector<size_t> slots;    // route slot (token * k + j) for each token
};

// Qwen38Expert::forward_projections{,_batch} with BF16 weights
// (src/models/qwen3_8/expert.rs:137-312): g = bf16(gate x), u = bf16(up x),
// a = bf16(bf16(silu(g)) * u), y = bf16(down a).
int qwen_expert(Pool &p, const urbo_matrix *m, size_t H, size_t I, const float *x, size_t n,
                float *y) {
    std::vector<float> g(n * I), u(n * I), a(n * I);
    int st = qwen_linear(p, m[0].data, I, H, x, n, g.data());
    if (st) return st;
    st = qwen_linear(p, m[1].data, I, H, x, n, u.data());
    if (st) return st;
    for (size_t i = 0; i < n * I; ++i) {
        float ag;
        if (!rne_bf16(silu_f(g[i]), &ag)) return URBO_NONFINITE;
        float v = ag * u[i];
        if (!std::isfinite(v)) return URBO_NONFINITE;
        a[i] = v;
    }
    st = urbo_round_to_bf16_in_place(a.data(), n * I);
    if (st) return st;
    return qwen_linear(p, m[2].data, H, I, a.data(), n, y);
}

// GatedMlp::forward (src/model/mlp.rs:90-99): down(silu(gate x) * up x), f32 in between,
// each projection through WeightMatrix::matvec (matmul_rows for a token group).
int gated_mlp(Pool &p, int format, const urbo_matrix *m, size_t H, size_t I, const float *x,
              size_t n, float *y) {
    std::vector<float> g(n * I), u(n * I), a(n * I);
    int st = weight_matmul(p, format, m[0].data, m[0].scales, I, H, x, n, g.data());
    if (st) return st;
    st = weight_matmul(p, format, m[1].data, m[1].scales, I, H, x, n, u.data());
    if (st) return st;
    for (size_t i = 0; i < n * I; ++i) a[i] = silu_f(g[i]) * u[i];
    return weight_matmul(p, format, m[2].data, m[2].scales, H, I, a.data(), n, y);
}

// Hy4 routed expert on quantized activations q [n, H] (src/models/hy4/expert.rs:373-392 and
// activate_gate_up :664-680): gate/up through WeightMatrix::matvec, each rounded to BF16;
// bounded_swiglu (deepseek_v4/math.rs:526-548): g' = min(g, limit), u' = clamp(u, +-limit),
// a = g' / (1 + exp(-g')) * u'; a <- simulate_e4m3_activation(a, 32) per token;
// y = bf16(down . a).
int hy4_routed(Pool &p, int format, const urbo_matrix *m, size_t H, size_t I, const float *q,
               size_t n, float limit, float *y) {
    std::vector<float> g(n * I), u(n * I), a(n * I);
    int st = weight_matmul(p, format, m[0].data, m[0].scales, I, H, q, n, g.data());
    if (st) return st;
    st = weight_matmul(p, format, m[1].data, m[1].scales, I, H, q, n, u.data());
    if (st) return st;
    if ((st = urbo_round_to_bf16_in_place(g.data(), n * I))) return st;
    if ((st = urbo_round_to_bf16_in_place(u.data(), n * I))) return st;
    if ((st = urbo_bounded_swiglu(g.data(), u.data(), n * I, limit, a.data()))) return st;
    for (size_t t = 0; t < n; ++t)
        if ((st = urbo_simulate_e4m3_activation(&a[t * I], I, 32))) return st;
    st = weight_matmul(p, format, m[2].data, m[2].scales, H, I, a.data(), n, y);
    if (st) return st;
    return urbo_round_to_bf16_in_place(y, n * H);
}

// Hy4 shared DenseMlp::forward (src/models/hy4/runtime.rs:1311-1322, mx_linear :2425-2442) on
// quantized activations q [n, H]: g = bf16(gate . q), u = bf16(up . q), a = bf16(silu(g) u),
// y = bf16(down . simulate_e4m3_activation(a, 32)).
int hy4_shared(Pool &p, int format, const urbo_matrix *m, size_t H, size_t I, const float *q,
               size_t n, float *y) {
    std::vector<float> g(n * I), u(n * I), a(n * I);
    int st = weight_matmul(p, format, m[0].data, m[0].scales, I, H, q, n, g.data());
    if (st) return st;
    st = weight_matmul(p, format, m[1].data, m[1].scales, I, H, q, n, u.data());
    if (st) return st;
    if ((st = urbo_round_to_bf16_in_place(g.data(), n * I))) return st;
    if ((st = urbo_round_to_bf16_in_place(u.data(), n * I))) return st;
    for (size_t i = 0; i < n * I; ++i) a[i] = silu_f(g[i]) * u[i];
    if ((st = urbo_round_to_bf16_in_place(a.data(), n * I))) return st;
    for (size_t t = 0; t < n; ++t)
        if ((st = urbo_simulate_e4m3_activation(&a[t * I], I, 32))) return st;
    st = weight_matmul(p, format, m[2].data, m[2].scales, H, I, a.data(), n, y);
    if (st) return st;
    return urbo_round_to_bf16_in_place(y, n * H);
}

// mx_activation (src/models/hy4/runtime.rs:2430-2434) of n tokens [n, H].
int hy4_quantize(const float *x, size_t n, size_t H, std::vector<float> &q) {
    q.assign(x, x + n * H);
    for (size_t t = 0; t < n; ++t) {
        int st = urbo_simulate_e4m3_activation(&q[t * H], H, 32);
        if (st) return st;
    }
    return URBO_OK;
}

// The DeepSeek routed expert on its input rows xin [n, H] (the simulated E4M3 activation for MX
// weights, the plain input otherwise):
//   V4.1 Expert::forward_with_mx_input (src/models/deepseek_v41/runtime.rs:2243-2261):
//     projections through matvec_fp32_accum (deepseek_v41/math.rs:36-52), 32-wide blocks;
//   V4 DeepExpert::forward_with_mx_input{,_batch} (src/models/deepseek_v4/runtime.rs:3081-3155):
//     projections through WeightMatrix::matvec / matmul_rows (deepseek_v4/math.rs:130-158),
//     128-wide blocks.
// gate, up = linear_with_mx_activation(w1 / w3) (BF16-rounded for MX weights only);
// a = bounded_swiglu(gate, up, limit) times the route weight of each token when given (`w`,
// may be null: the shared expert); a -> BF16; y = linear(w2, a): MX weights read
// simulate_e4m3_activation(a, block) and round y to BF16, other weights read a as it is.
int dsv_expert(Pool &p, bool v41, int format, const urbo_matrix *m, size_t H, size_t I,
               const float *xin, size_t n, float limit, const float *w, float *y) {
    const bool mx = format == URBO_FMT_MXFP4 || format == URBO_FMT_MXFP8;
    const size_t block = v41 ? 32 : 128;
    auto mm = [&](const urbo_matrix &mat, size_t rows, size_t cols, const float *x, float *out) {
        return v41 ? weight_matmul_fp32_accum(p, format, mat.data, mat.scales, rows, cols, x, n,
                                              out)
                   : weight_matmul(p, format, mat.data, mat.scales, rows, cols, x, n, out);
    };
    std::vector<float> g(n * I), u(n * I), a(n * I);
    int st = mm(m[0], I, H, xin, g.data());
    if (st) return st;
    if ((st = mm(m[1], I, H, xin, u.data()))) return st;
    if (mx && (st = urbo_round_to_bf16_in_place(g.data(), n * I))) return st;
    if (mx && (st = urbo_round_to_bf16_in_place(u.data(), n * I))) return st;
    if ((st = urbo_bounded_swiglu(g.data(), u.data(), n * I, limit, a.data()))) return st;
    if (w)
        for (size_t t = 0; t < n; ++t) {
            // v4 runtime.rs:3089-3094, v4.1 runtime.rs:2085-2090: a non-finite or negative
            // route weight is rejected
            if (!std::isfinite(w[t]) || w[t] < 0.0f) return URBO_INVALID_GEOMETRY;
            for (size_t i = 0; i < I; ++i) a[t * I + i] *= w[t];
        }
    if ((st = urbo_round_to_bf16_in_place(a.data(), n * I))) return st;
    if (mx)
        for (size_t t = 0; t < n; ++t)
            if ((st = urbo_simulate_e4m3_activation(&a[t * I], I, block))) return st;
    if ((st = mm(m[2], H, I, a.data(), y))) return st;
    return mx ? urbo_round_to_bf16_in_place(y, n * H) : URBO_OK;
}

// mx_activation / prepare_mx_activation of n tokens [n, H] per `block` values.
int quantize_rows(const float *x, size_t n, size_t H, size_t block, std::vector<float> &q) {
    q.assign(x, x + n * H);
    for (size_t t = 0; t < n; ++t) {
        int st = urbo_simulate_e4m3_activation(&q[t * H], H, block);
        if (st) return st;
    }
    return URBO_OK;
}

}  // namespace

int urbo_hy4_expert(int format, const urbo_matrix *m, uint32_t H, uint32_t I, const float *x,
                    uint32_t n, float swiglu_limit, float *y, int threads) {
    if (H == 0 || I == 0 || n == 0) return URBO_SHAPE;
    if (format != URBO_FMT_MXFP4 && format != URBO_FMT_MXFP8) return URBO_SHAPE;
    std::vector<float> q;
    int st = hy4_quantize(x, n, H, q);
    if (st) return st;
    Pool &p = pool(threads);
    return swiglu_limit > 0.0f ? hy4_routed(p, format, m, H, I, q.data(), n, swiglu_limit, y)
                               : hy4_shared(p, format, m, H, I, q.data(), n, y);
}

int urbo_dsv41_expert(int format, const urbo_matrix *m, uint32_t H, uint32_t I, const float *x,
                      uint32_t n, float swiglu_limit, const float *route_weights, float *y,
                      int threads) {
    if (H == 0 || I == 0 || n == 0) return URBO_SHAPE;
    if (format != URBO_FMT_MXFP4 && format != URBO_FMT_MXFP8) return URBO_SHAPE;
    std::vector<float> q;
    int st = hy4_quantize(x, n, H, q);
    if (st) return st;
    return dsv_expert(pool(threads), true, format, m, H, I, q.data(), n, swiglu_limit,
                      route_weights, y);
}

int urbo_dsv4_expert(int format, const urbo_matrix *m, uint32_t H, uint32_t I, const float *x,
                     uint32_t n, float swiglu_limit, const float *route_weights, float *y,
                     int threads) {
    if (H == 0 || I == 0 || n == 0) return URBO_SHAPE;
    if (format < URBO_FMT_BF16 || format > URBO_FMT_F32) return URBO_SHAPE;
    if (!all_finite(x, (size_t)n * H)) return URBO_NONFINITE;
    std::vector<float> q;
    const bool mx = format == URBO_FMT_MXFP4 || format == URBO_FMT_MXFP8;
    if (mx) {
        int st = quantize_rows(x, n, H, 128, q);
        if (st) return st;
    }
    return dsv_expert(pool(threads), false, format, m, H, I, mx ? q.data() : x, n, swiglu_limit,
                      route_weights, y);
}

int urbo_gated_mlp(int format, const urbo_matrix *m, uint32_t H, uint32_t I, const float *x,
                   uint32_t n, float *y, int threads) {
    if (H == 0 || I == 0 || n == 0) return URBO_SHAPE;
    return gated_mlp(pool(threads), format, m, H, I, x, n, y);
}

int urbo_qwen_expert(const urbo_matrix *m, uint32_t H, uint32_t I, const float *x, uint32_t n,
                     float *y, int threads) {
    if (H == 0 || I == 0 || n == 0) return URBO_SHAPE;
    if (!all_finite(x, (size_t)n * H)) return URBO_NONFINITE;
    return qwen_expert(pool(threads), m, H, I, x, n, y);
}

int urbo_moe_forward(const urbo_layer *L, const float *x, uint32_t T, float *y, int32_t *ids,
                     float *weights, float *logits_out, int threads) {
    return urbo_moe_forward_tokens(L, x, nullptr, T, y, ids, weights, logits_out, threads);
}

int urbo_moe_forward_tokens(const urbo_layer *L, const float *x, const uint32_t *tokens,
                            uint32_t T, float *y, int32_t *ids, float *weights,
                            float *logits_out, int threads) {
    const size_t H = L->hidden, E = L->n_experts, K = L->top_k, I = L->intermediate;
    if (H == 0 || E == 0 || I == 0 || T == 0) return URBO_SHAPE;
    if (K == 0 || K > E) return URBO_INVALID_GEOMETRY;
    const bool qwen = L->composition == URBO_COMPOSE_QWEN36;
    const bool v4 = L->composition == URBO_COMPOSE_DSV4;
    const bool v41 = L->composition == URBO_COMPOSE_DSV41;
    const bool dsv = v41 || v4;
    const bool hy4 = L->composition == URBO_COMPOSE_HY4;
    const bool mxa = hy4 || v41;  // MX projections only
    auto is_mx = [](int f) { return f == URBO_FMT_MXFP4 || f == URBO_FMT_MXFP8; };
    // hash experts (the first num_hash_layers layers of DeepSeek V4, runtime.rs:2664-2681): a
    // [hash_vocab, K] table row per token id; only with route_sqrt_softplus
    if (L->hash_experts && (L->router != URBO_ROUTER_SQRT_SOFTPLUS || !tokens)) return URBO_SHAPE;
    if (v4 && !(L->swiglu_limit > 0.0f && std::isfinite(L->swiglu_limit)))
        return URBO_INVALID_GEOMETRY;
    if (qwen && (L->expert_format != URBO_FMT_BF16 ||
                 (L->shared_intermediate &&
                  (L->shared_format != URBO_FMT_BF16 || !L->shared_expert_gate || !L->shared))))
        return URBO_SHAPE;
    if (mxa && (L->expert_format == URBO_FMT_BF16 ||
                (L->shared_intermediate && L->shared_format == URBO_FMT_BF16)))
        return URBO_SHAPE;
    if (mxa && !(L->swiglu_limit > 0.0f && std::isfinite(L->swiglu_limit)))
        return URBO_INVALID_GEOMETRY;
    Pool &p = pool(threads);
    if (!all_finite(x, (size_t)T * H)) return URBO_NONFINITE;

    // Router logits: Qwen `linear(router)` (qwen3_8/math.rs:10-26, FP32 GEMV + BF16), DeepSeek
    // V4.1 `router.matvec_fp32_accum` (deepseek_v41/runtime.rs:2136, FP32 GEMV), GLM and Hy4
    // `router.matvec` (ordered f64, bf16.rs:121-216).
    // DeepSeek V4 `linear(router)` on its BF16 or F32 router is the ordered-f64 matvec too
    // (deepseek_v4/math.rs:106-115; bf16.rs:121-216, matrix.rs:236-259).
    std::vector<float> logits((size_t)T * E);
    const uint8_t *rw = (const uint8_t *)L->router_weight;
    int st = qwen  ? qwen_linear(p, rw, E, H, x, T, logits.data())
             : v41 ? bf16_matmul_fp32(p, rw, E, H, x, T, logits.data())
             : (v4 && L->router_weight_f32)
                 ? weight_matmul(p, URBO_FMT_F32, (const uint8_t *)L->router_weight_f32, nullptr,
                                 E, H, x, T, logits.data())
                 : weight_matmul(p, URBO_FMT_BF16, rw, nullptr, E, H, x, T, logits.data());
    if (st) return st;
    if (logits_out) std::memcpy(logits_out, logits.data(), logits.size() * 4);

    // Routes, ranking order per token.
    std::vector<int32_t> rid((size_t)T * K);
    std::vector<float> rw8((size_t)T * K);
    for (size_t t = 0; t < T; ++t) {
        const float *lt = logits.data() + t * E;
        if (L->router == URBO_ROUTER_SOFTMAX_TOPK)
            st = urbo_route_softmax_top_k(lt, E, K, &rid[t * K], &rw8[t * K]);
        else if (L->router == URBO_ROUTER_SQRT_SOFTPLUS) {
            const int64_t *row = nullptr;
            if (L->hash_experts) {
                // load_i64_matrix_row(tid2eid, token, vocab, K) (runtime.rs:2665-2671)
                if (tokens[t] >= L->hash_vocab) return URBO_SHAPE;
                row = L->hash_experts + (size_t)tokens[t] * K;
            }
            st = urbo_route_sqrt_softplus_hashed(lt, L->correction_bias, row, E, K,
                                                 L->routed_scaling_factor, &rid[t * K],
                                                 &rw8[t * K], nullptr);
        }
        else
            st = urbo_route_noaux_tc(lt, L->correction_bias, E, K, L->n_group, L->topk_group,
                                     L->normalize, L->routed_scaling_factor, &rid[t * K],
                                     &rw8[t * K], nullptr);
        if (st) return st;
        // Qwen3.6 rounds every route weight to BF16 (qwen3_6/runtime.rs:1085-1090, 1233-1238).
        if (qwen)
            for (size_t j = 0; j < K; ++j)
                if (!rne_bf16(rw8[t * K + j], &rw8[t * K + j])) return URBO_NONFINITE;
    }
    if (ids) std::memcpy(ids, rid.data(), rid.size() * 4);
    if (weights) std::memcpy(weights, rw8.data(), rw8.size() * 4);

    // Permutation: groups by ascending expert id, tokens ascending inside a group.
    std::vector<Group> groups;
    {
        std::vector<std::vector<std::pair<size_t, size_t>>> by(E);
        for (size_t t = 0; t < T; ++t)
            for (size_t j = 0; j < K; ++j) by[rid[t * K + j]].push_back({t, t * K + j});
        for (size_t e = 0; e < E; ++e) {
            if (by[e].empty()) continue;
            Group g; g.expert = e;
            for (auto &ts : by[e]) { g.tokens.push_back(ts.first); g.slots.push_back(ts.second); }
            groups.push_back(std::move(g));
        }
    }
    // Hy4: one E4M3 activation per token shared by every routed expert and the shared expert
    // (src/models/hy4/runtime.rs:1397, 1311-1312).
    // DeepSeek V4 prepare_mx_activation (runtime.rs:2691-2693): 128-wide blocks, read by the
    // MX matrices only.
    std::vector<float> qx;
    if (mxa && (st = hy4_quantize(x, T, H, qx))) return st;
    if (v4 && (is_mx(L->expert_format) || (L->shared_intermediate && is_mx(L->shared_format))) &&
        (st = quantize_rows(x, T, H, 128, qx)))
        return st;
    const float *xe = mxa || (v4 && is_mx(L->expert_format)) ? qx.data() : x;
    const float *xs = mxa || (v4 && is_mx(L->shared_format)) ? qx.data() : x;
    // Expert outputs per route slot.
    std::vector<float> out((size_t)T * K * H);
    for (const Group &g : groups) {
        size_t n = g.tokens.size();
        std::vector<float> xin(n * H), yo(n * H);
        for (size_t i = 0; i < n; ++i)
            std::memcpy(&xin[i * H], xe + g.tokens[i] * H, H * 4);
        const urbo_matrix *m = L->experts + g.expert * 3;
        if (!m[0].data || !m[1].data || !m[2].data) return URBO_SHAPE;  // expert not supplied
        std::vector<float> wr;
        if (dsv)
            for (size_t slot : g.slots) wr.push_back(rw8[slot]);
        st = qwen  ? qwen_expert(p, m, H, I, xin.data(), n, yo.data())
             : hy4 ? hy4_routed(p, L->expert_format, m, H, I, xin.data(), n, L->swiglu_limit,
                                yo.data())
             : dsv ? dsv_expert(p, v41, L->expert_format, m, H, I, xin.data(), n,
                                L->swiglu_limit, wr.data(), yo.data())
                   : gated_mlp(p, L->expert_format, m, H, I, xin.data(), n, yo.data());
        if (st) return st;
        for (size_t i = 0; i < n; ++i)
            std::memcpy(&out[g.slots[i] * H], &yo[i * H], H * 4);
    }

    if (qwen) {
        // accumulate_routed_expert in ascending expert id (qwen3_6/runtime.rs:1239-1241,
        // 1398-1415): c = bf16(w * v), acc = bf16(acc + c); final finite check (:1462-1467).
        for (size_t t = 0; t < T; ++t) {
            std::vector<size_t> order(K);
            for (size_t j = 0; j < K; ++j) order[j] = j;
            std::stable_sort(order.begin(), order.end(), [&](size_t a, size_t b) {
                return rid[t * K + a] < rid[t * K + b];
            });
            float *yt = y + t * H;
            for (size_t h = 0; h < H; ++h) yt[h] = 0.0f;
            for (size_t j : order) {
                const float w = rw8[t * K + j];
                const float *v = &out[(t * K + j) * H];
                for (size_t h = 0; h < H; ++h) {
                    float c;
                    if (!rne_bf16(w * v[h], &c)) return URBO_NONFINITE;
                    float acc = yt[h] + c;
                    if (!rne_bf16(acc, &yt[h])) return URBO_NONFINITE;
                }
            }
        }
        if (L->shared_intermediate) {
            // finish_ordered_moe (qwen3_6/runtime.rs:1417-1468; batched :1169-1211): the shared
            // Qwen38Expert, its gate linear(shared_expert_gate) (FP32 GEMV + BF16), scale =
            // bf16(sigmoid(gate)) in the two-branch form, acc = bf16(acc + bf16(scale * s)).
            const size_t Is = L->shared_intermediate;
            std::vector<float> sh((size_t)T * H), gate(T);
            st = qwen_expert(p, L->shared, H, Is, x, T, sh.data());
            if (st) return st;
            st = qwen_linear(p, (const uint8_t *)L->shared_expert_gate, 1, H, x, T, gate.data());
            if (st) return st;
            for (size_t t = 0; t < T; ++t) {
                const float g = gate[t];
                if (!std::isfinite(g)) return URBO_NONFINITE;
                float scale;
                if (g >= 0.0f) {
                    scale = 1.0f / (1.0f + ::expf(-g));
                } else {
                    const float e = ::expf(g);
                    scale = e / (1.0f + e);
                }
                if (!rne_bf16(scale, &scale)) return URBO_NONFINITE;
                float *yt = y + t * H;
                const float *s = &sh[t * H];
                for (size_t h = 0; h < H; ++h) {
                    float c;
                    if (!rne_bf16(scale * s[h], &c)) return URBO_NONFINITE;
                    if (!rne_bf16(yt[h] + c, &yt[h])) return URBO_NONFINITE;
                }
            }
        }
        return URBO_OK;
    }

    if (mxa || v4) {
        // Hy4 MoeWeights::forward (src/models/hy4/runtime.rs:1387-1445): f32 sum of w * y over
        // the routes in ascending expert id, plus the shared expert, rounded to BF16.  DeepSeek
        // V4.1 (deepseek_v41/runtime.rs:1963-2019) and V4 (deepseek_v4/runtime.rs:2498-2653) the
        // same with the route weight already applied inside each expert (the sum adds y).
        std::vector<float> sh;
        if (L->shared_intermediate) {
            sh.resize((size_t)T * H);
            st = hy4 ? hy4_shared(p, L->shared_format, L->shared, H, L->shared_intermediate,
                                  qx.data(), T, sh.data())
                     : dsv_expert(p, v41, L->shared_format, L->shared, H, L->shared_intermediate,
                                  xs, T, L->swiglu_limit, nullptr, sh.data());
            if (st) return st;
        }
        for (size_t t = 0; t < T; ++t) {
            std::vector<size_t> order(K);
            for (size_t j = 0; j < K; ++j) order[j] = j;
            std::stable_sort(order.begin(), order.end(), [&](size_t a, size_t b) {
                return rid[t * K + a] < rid[t * K + b];
            });
            float *yt = y + t * H;
            for (size_t h = 0; h < H; ++h) yt[h] = 0.0f;
            for (size_t j : order) {
                const float w = rw8[t * K + j];
                const float *v = &out[(t * K + j) * H];
                if (dsv)
                    for (size_t h = 0; h < H; ++h) yt[h] += v[h];
                else
                    for (size_t h = 0; h < H; ++h) yt[h] += w * v[h];
            }
            if (!sh.empty())
                for (size_t h = 0; h < H; ++h) yt[h] += sh[t * H + h];
        }
        return urbo_round_to_bf16_in_place(y, (size_t)T * H);
    }

    // GLM: shared expert first (moe.rs:162-165), then f64 accumulation in ranking order.
    std::vector<double> acc((size_t)T * H, 0.0);
    if (L->shared_intermediate) {
        std::vector<float> sh((size_t)T * H);
        st = gated_mlp(p, L->shared_format, L->shared, H, L->shared_intermediate, x, T, sh.data());
        if (st) return st;
        for (size_t i = 0; i < sh.size(); ++i) acc[i] = (double)sh[i];
    }
    for (size_t t = 0; t < T; ++t)
        for (size_t j = 0; j < K; ++j) {
            const double w = (double)rw8[t * K + j];
            const float *v = &out[(t * K + j) * H];
            double *a = &acc[t * H];
            for (size_t h = 0; h < H; ++h) a[h] += w * (double)v[h];
        }
    for (size_t i = 0; i < acc.size(); ++i) y[i] = (float)acc[i];
    return URBO_OK;
}

}  // extern "C"
