// oracle_kv.cpp — scalar CPU restatement of AtomFlow's KV-cache hot path.
//
// TEST INFRASTRUCTURE (see oracle_kv.h): the checker for libatomflow_kv.so and
// the timed CPU baseline; never linked into the product.
//
// Build with -ffp-contract=off: the reference's RoPE expression
// `x * cos - y * sin` (src/kernel/rope.cu:34-35) is defined here as two fp32
// products and one fp32 subtraction, each rounded, then one fp32->fp16 RNE.
#include "oracle_kv.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

namespace {

inline uint32_t f2u(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}
inline float u2f(uint32_t u) {
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

}  // namespace

// Exported functions take C linkage from their declarations in oracle_kv.h.

// ---- IEEE binary16 <-> binary32, round to nearest even ----------------------
// The reference casts with `(half)float` / __float2half, both round-to-nearest-
// even (src/kernel/rope.cu:34-35, src/kernel/tiled_attention.cu:268).
uint16_t ok_f32_to_f16(float f) {
    const uint32_t u = f2u(f);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const uint32_t absu = u & 0x7fffffffu;
    if (absu >= 0x7f800000u) {  // inf or NaN
        if (absu == 0x7f800000u) return uint16_t(sign | 0x7c00u);
        return uint16_t(sign | 0x7e00u | ((absu >> 13) & 0x3ffu));  // quiet NaN, keep payload bits
    }
    const int32_t exp = int32_t(absu >> 23) - 127;  // unbiased
    if (exp > 15) return uint16_t(sign | 0x7c00u);   // overflow -> inf (>= 65536)
    if (exp >= -14) {
        // normal half: 10 mantissa bits kept, 13 dropped
        uint32_t mant = absu & 0x7fffffu;
        uint32_t h = (uint32_t(exp + 15) << 10) | (mant >> 13);
        const uint32_t rem = mant & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1;  // carry may bump exponent
        return uint16_t(sign | h);  // h == 0x7c00 after carry means overflow to inf: correct
    }
    // subnormal half (or zero): value = m * 2^-24, m in [0, 1024]
    if (exp < -25) return uint16_t(sign);  // < 2^-25: rounds to zero (2^-25 exactly is a tie -> 0)
    // value = mant * 2^(exp-23) = mant * 2^(exp+1) units of 2^-24 -> shift right by -(exp+1)
    const uint32_t mant = (absu & 0x7fffffu) | 0x800000u;  // 24-bit significand
    const int shift = -exp - 1;                            // 14 .. 24
    const uint32_t q = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t half_ulp = 1u << (shift - 1);
    uint32_t h = q;
    if (rem > half_ulp || (rem == half_ulp && (h & 1u))) h += 1;
    return uint16_t(sign | h);
}

float ok_f16_to_f32(uint16_t h) {
    const uint32_t sign = uint32_t(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    if (e == 0) {
        if (m == 0) return u2f(sign);
        // subnormal: m * 2^-24 is exact in float
        float v = float(m) * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

void ok_f32_to_f16_array(const float* src, uint16_t* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = ok_f32_to_f16(src[i]);
}
void ok_f16_to_f32_array(const uint16_t* src, float* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = ok_f16_to_f32(src[i]);
}

// ---- a1: RoPE table — src/kernel/helpers.cu:94-113 --------------------------
// theta = s / pow(base, 2.0f*i/head_dim) with the float overloads of std::pow,
// std::cos, std::sin (all operands are float at helpers.cu:102-104).
void ok_rope_table(float* cos_out, float* sin_out, int max_seq, int head_dim, float base) {
    const int half_dim = head_dim / 2;
    for (int s = 0; s < max_seq; ++s) {
        for (int i = 0; i < half_dim; ++i) {
            const float expo = 2.0f * float(i) / float(head_dim);
            const float theta = float(s) / std::pow(base, expo);
            cos_out[size_t(s) * half_dim + i] = std::cos(theta);
            sin_out[size_t(s) * half_dim + i] = std::sin(theta);
        }
    }
}

// ---- a2: RoPE — src/kernel/rope.cu:11-46 ------------------------------------
// For token p (blockIdx.x) and pair d (threadIdx.x < head_dim/2): the pair
// (d, d+head_dim/2) of every Q head, then of every K head, rotated by table
// row p. Q rows are q_head_num*head_dim apart, K rows kv_head_num*head_dim.
static inline void rotate_pair(uint16_t* x_ptr, uint16_t* y_ptr, float c, float s) {
    const float x = ok_f16_to_f32(*x_ptr);
    const float y = ok_f16_to_f32(*y_ptr);
    const float xc = x * c;
    const float ys = y * s;
    const float xs = x * s;
    const float yc = y * c;
    *x_ptr = ok_f32_to_f16(xc - ys);
    *y_ptr = ok_f32_to_f16(xs + yc);
}

void ok_rope(uint16_t* q, uint16_t* k, const float* cos_cache, const float* sin_cache,
             int seq_len, int kv_head_num, int q_head_num, int head_dim) {
    const int half_dim = head_dim / 2;
    for (int p = 0; p < seq_len; ++p) {
        for (int d = 0; d < half_dim; ++d) {
            const float c = cos_cache[size_t(p) * half_dim + d];
            const float s = sin_cache[size_t(p) * half_dim + d];
            for (int h = 0; h < q_head_num; ++h) {
                uint16_t* cur = q + (size_t(p) * q_head_num + h) * head_dim;
                rotate_pair(cur + d, cur + d + half_dim, c, s);
            }
            for (int h = 0; h < kv_head_num; ++h) {
                uint16_t* cur = k + (size_t(p) * kv_head_num + h) * head_dim;
                rotate_pair(cur + d, cur + d + half_dim, c, s);
            }
        }
    }
}

// ---- a3: KV write — src/kernel/helpers.cu:126-139 ---------------------------
void ok_write_kv_cache(const uint16_t* qkv_out, uint16_t* k_cache, uint16_t* v_cache,
                       int current_pos, int q_dim, int kv_dim) {
    std::memcpy(k_cache + size_t(current_pos) * kv_dim, qkv_out + q_dim, size_t(kv_dim) * 2);
    std::memcpy(v_cache + size_t(current_pos) * kv_dim, qkv_out + q_dim + kv_dim,
                size_t(kv_dim) * 2);
}

// ---- a2+a3: the engine's sequence — src/core/engine.cu:326-355 --------------
// launch_rope on (q = qkv_out, k = qkv_out + Q_DIM) with the table pointers
// advanced by pos*head_dim/2 and seq_len 1, then launch_write_kv_cache(pos).
void ok_rope_append(uint16_t* qkv_out, uint16_t* k_cache, uint16_t* v_cache,
                    const float* cos_table, const float* sin_table, int pos, int n_q_heads,
                    int n_kv_heads, int head_dim) {
    const int q_dim = n_q_heads * head_dim;
    const int kv_dim = n_kv_heads * head_dim;
    const size_t off = size_t(pos) * (head_dim / 2);
    ok_rope(qkv_out, qkv_out + q_dim, cos_table + off, sin_table + off, 1, n_kv_heads, n_q_heads,
            head_dim);
    ok_write_kv_cache(qkv_out, k_cache, v_cache, pos, q_dim, kv_dim);
}

// ---- a5: decode attention — src/kernel/tiled_attention.cu:196-269 ----------
// Per query head h (one block of head_dim threads in the reference):
//   kv_h = h*n_kv_heads/n_q_heads                               (:208)
//   score[t] = tree_sum_d(q[d]*k[t,d]) * (1/sqrt(head_dim))     (:224-240)
//   max, exp(score - max), serial sum, multiply by 1/sum        (:244-258)
//   out[d] = sum_t p[t]*v[t,d] in fp32, serial in t, fp16 RNE   (:262-268)
// Elements are read through the accessors so the FP8 pool shares this code.
template <typename KF, typename VF>
static void attention_head_f32(const uint16_t* q_h, int seq_len, int head_dim, KF kval, VF vval,
                               uint16_t* out_h, std::vector<float>& red,
                               std::vector<float>& scores) {
    const float inv_sqrt_hd = 1.0f / std::sqrt(float(head_dim));
    red.resize(head_dim);
    scores.resize(seq_len);
    for (int t = 0; t < seq_len; ++t) {
        for (int d = 0; d < head_dim; ++d) red[d] = ok_f16_to_f32(q_h[d]) * kval(t, d);
        for (int stride = head_dim >> 1; stride > 0; stride >>= 1)
            for (int d = 0; d < stride; ++d) red[d] += red[d + stride];
        scores[t] = red[0] * inv_sqrt_hd;
    }
    float max_s = -1e38f;
    for (int t = 0; t < seq_len; ++t) max_s = std::fmax(max_s, scores[t]);
    float sum_exp = 0.0f;
    for (int t = 0; t < seq_len; ++t) {
        scores[t] = std::exp(scores[t] - max_s);
        sum_exp += scores[t];
    }
    const float inv_sum = 1.0f / sum_exp;
    for (int t = 0; t < seq_len; ++t) scores[t] *= inv_sum;
    for (int d = 0; d < head_dim; ++d) {
        float acc = 0.0f;
        for (int t = 0; t < seq_len; ++t) acc += scores[t] * vval(t, d);
        out_h[d] = ok_f32_to_f16(acc);
    }
}

static void attention_heads_range(const uint16_t* q, const uint16_t* k_cache,
                                  const uint16_t* v_cache, uint16_t* out, int seq_len,
                                  int head_dim, int n_q_heads, int n_kv_heads, int h_begin,
                                  int h_end) {
    const size_t row = size_t(n_kv_heads) * head_dim;
    std::vector<float> red, scores;
    for (int h = h_begin; h < h_end; ++h) {
        const int kv_h = h * n_kv_heads / n_q_heads;
        const uint16_t* kb = k_cache + size_t(kv_h) * head_dim;
        const uint16_t* vb = v_cache + size_t(kv_h) * head_dim;
        auto kf = [&](int t, int d) { return ok_f16_to_f32(kb[size_t(t) * row + d]); };
        auto vf = [&](int t, int d) { return ok_f16_to_f32(vb[size_t(t) * row + d]); };
        attention_head_f32(q + size_t(h) * head_dim, seq_len, head_dim, kf, vf,
                           out + size_t(h) * head_dim, red, scores);
    }
}

void ok_cached_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                         uint16_t* out, int seq_len, int head_dim, int n_q_heads,
                         int n_kv_heads) {
    attention_heads_range(q, k_cache, v_cache, out, seq_len, head_dim, n_q_heads, n_kv_heads, 0,
                          n_q_heads);
}

void ok_cached_attention_mt(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                            uint16_t* out, int seq_len, int head_dim, int n_q_heads,
                            int n_kv_heads, int n_threads) {
    if (n_threads <= 1) {
        ok_cached_attention(q, k_cache, v_cache, out, seq_len, head_dim, n_q_heads, n_kv_heads);
        return;
    }
    if (n_threads > n_q_heads) n_threads = n_q_heads;
    std::vector<std::thread> pool;
    for (int i = 0; i < n_threads; ++i) {
        const int hb = n_q_heads * i / n_threads, he = n_q_heads * (i + 1) / n_threads;
        pool.emplace_back(attention_heads_range, q, k_cache, v_cache, out, seq_len, head_dim,
                          n_q_heads, n_kv_heads, hb, he);
    }
    for (auto& t : pool) t.join();
}

void ok_cached_attention_f64(const uint16_t* q, const uint16_t* k_cache,
                             const uint16_t* v_cache, double* out, int seq_len, int head_dim,
                             int n_q_heads, int n_kv_heads) {
    const size_t row = size_t(n_kv_heads) * head_dim;
    const double inv_sqrt_hd = 1.0 / std::sqrt(double(head_dim));
    std::vector<double> scores(seq_len);
    for (int h = 0; h < n_q_heads; ++h) {
        const int kv_h = h * n_kv_heads / n_q_heads;
        const uint16_t* qh = q + size_t(h) * head_dim;
        for (int t = 0; t < seq_len; ++t) {
            double dot = 0.0;
            for (int d = 0; d < head_dim; ++d)
                dot += double(ok_f16_to_f32(qh[d])) *
                       double(ok_f16_to_f32(k_cache[size_t(t) * row + size_t(kv_h) * head_dim + d]));
            scores[t] = dot * inv_sqrt_hd;
        }
        double m = -1e300;
        for (int t = 0; t < seq_len; ++t) m = std::fmax(m, scores[t]);
        double l = 0.0;
        for (int t = 0; t < seq_len; ++t) {
            scores[t] = std::exp(scores[t] - m);
            l += scores[t];
        }
        for (int d = 0; d < head_dim; ++d) {
            double acc = 0.0;
            for (int t = 0; t < seq_len; ++t)
                acc += scores[t] *
                       double(ok_f16_to_f32(v_cache[size_t(t) * row + size_t(kv_h) * head_dim + d]));
            out[size_t(h) * head_dim + d] = acc / l;
        }
    }
}

// ---- b2: causal prefill attention — src/kernel/tiled_attention.cu:34-130 -------
// Per (query token i, head h), one block of head_dim threads in the reference:
//   kv_h = h*n_kv_heads/n_q_heads                                  (:55)
//   score[s] = serial_sum_d(q[d]*k[s,d]) * (1/sqrt(head_dim))     (:82-96)
//   for s < n_keys = min(i+1, seq_kv)                              (:82,:103)
//   max (from -1e38), p = exp(score - max), serial sum, p /= sum   (:101-116)
//   out[d] = sum_s p[s]*v[s,d] in fp32, serial in s, fp16 RNE      (:119-126)
// With a chunk start p0 the key count is min(p0 + i + 1, kv_len).
static void prefill_rows(const uint16_t* q, int q_stride, const uint16_t* k_cache,
                         const uint16_t* v_cache, uint16_t* out, int out_stride, int p0,
                         int i_begin, int i_end, int kv_len, int head_dim, int n_q_heads,
                         int n_kv_heads) {
    const size_t row = size_t(n_kv_heads) * head_dim;
    const float inv_sqrt_hd = 1.0f / std::sqrt(float(head_dim));
    std::vector<float> scores(kv_len);
    for (int i = i_begin; i < i_end; ++i) {
        const int n_keys = std::min(p0 + i + 1, kv_len);
        for (int h = 0; h < n_q_heads; ++h) {
            const int kv_h = h * n_kv_heads / n_q_heads;
            const uint16_t* qh = q + size_t(i) * q_stride + size_t(h) * head_dim;
            for (int t = 0; t < n_keys; ++t) {
                const uint16_t* kt = k_cache + size_t(t) * row + size_t(kv_h) * head_dim;
                float score = 0.0f;
                for (int d = 0; d < head_dim; ++d)
                    score += ok_f16_to_f32(qh[d]) * ok_f16_to_f32(kt[d]);
                scores[t] = score * inv_sqrt_hd;
            }
            float max_s = -1e38f;
            for (int t = 0; t < n_keys; ++t) max_s = std::fmax(max_s, scores[t]);
            float sum_exp = 0.0f;
            for (int t = 0; t < n_keys; ++t) {
                scores[t] = std::exp(scores[t] - max_s);
                sum_exp += scores[t];
            }
            for (int t = 0; t < n_keys; ++t) scores[t] /= sum_exp;
            uint16_t* oh = out + size_t(i) * out_stride + size_t(h) * head_dim;
            for (int d = 0; d < head_dim; ++d) {
                float acc = 0.0f;
                for (int t = 0; t < n_keys; ++t)
                    acc += scores[t] *
                           ok_f16_to_f32(v_cache[size_t(t) * row + size_t(kv_h) * head_dim + d]);
                oh[d] = ok_f32_to_f16(acc);
            }
        }
    }
}

void ok_prefill_attention(const uint16_t* q, int q_stride, const uint16_t* k_cache,
                          const uint16_t* v_cache, uint16_t* out, int out_stride, int p0, int n,
                          int kv_len, int head_dim, int n_q_heads, int n_kv_heads, int n_threads) {
    if (n_threads <= 1 || n < 2) {
        prefill_rows(q, q_stride, k_cache, v_cache, out, out_stride, p0, 0, n, kv_len, head_dim,
                     n_q_heads, n_kv_heads);
        return;
    }
    if (n_threads > n) n_threads = n;
    // Rows near the end attend more keys: interleave blocks of rows over threads.
    std::vector<std::thread> pool;
    for (int w = 0; w < n_threads; ++w)
        pool.emplace_back([=] {
            for (int b = w * 8; b < n; b += 8 * n_threads)
                prefill_rows(q, q_stride, k_cache, v_cache, out, out_stride, p0, b,
                             std::min(b + 8, n), kv_len, head_dim, n_q_heads, n_kv_heads);
        });
    for (auto& t : pool) t.join();
}

void ok_prefill_attention_f64(const uint16_t* q, int q_stride, const uint16_t* k_cache,
                              const uint16_t* v_cache, double* out, int p0, int n, int kv_len,
                              int head_dim, int n_q_heads, int n_kv_heads) {
    const size_t row = size_t(n_kv_heads) * head_dim;
    const double inv_sqrt_hd = 1.0 / std::sqrt(double(head_dim));
    std::vector<double> scores(kv_len);
    for (int i = 0; i < n; ++i) {
        const int n_keys = std::min(p0 + i + 1, kv_len);
        for (int h = 0; h < n_q_heads; ++h) {
            const int kv_h = h * n_kv_heads / n_q_heads;
            const uint16_t* qh = q + size_t(i) * q_stride + size_t(h) * head_dim;
            double m = -1e300;
            for (int t = 0; t < n_keys; ++t) {
                double dot = 0.0;
                for (int d = 0; d < head_dim; ++d)
                    dot += double(ok_f16_to_f32(qh[d])) *
                           double(ok_f16_to_f32(k_cache[size_t(t) * row + size_t(kv_h) * head_dim + d]));
                scores[t] = dot * inv_sqrt_hd;
                m = std::fmax(m, scores[t]);
            }
            double l = 0.0;
            for (int t = 0; t < n_keys; ++t) {
                scores[t] = std::exp(scores[t] - m);
                l += scores[t];
            }
            double* oh = out + (size_t(i) * n_q_heads + h) * head_dim;
            for (int d = 0; d < head_dim; ++d) {
                double acc = 0.0;
                for (int t = 0; t < n_keys; ++t)
                    acc += scores[t] *
                           double(ok_f16_to_f32(v_cache[size_t(t) * row + size_t(kv_h) * head_dim + d]));
                oh[d] = acc / l;
            }
        }
    }
}

void ok_prefill_rope_append(uint16_t* qkv_out, int n, uint16_t* k_cache, uint16_t* v_cache,
                            const float* cos_table, const float* sin_table, int p0,
                            int n_q_heads, int n_kv_heads, int head_dim) {
    const size_t stride = size_t(n_q_heads + 2 * n_kv_heads) * head_dim;
    for (int i = 0; i < n; ++i)
        ok_rope_append(qkv_out + i * stride, k_cache, v_cache, cos_table, sin_table, p0 + i,
                       n_q_heads, n_kv_heads, head_dim);
}

// ---- a8: FP8 E4M3 codec ------------------------------------------------------
// OCP e4m3fn: s eeee mmm, bias 7, subnormal quantum 2^-9, max 448 (0x7E),
// 0x7F / 0xFF NaN, no infinities. The reference decodes with
// static_cast<float>(__nv_fp8_e4m3) (src/kernel/qkv_gemm.cu:80-81) and encodes
// with torch's float8_e4m3fn cast after clamping to +-448
// (tools/quantize_weights.py:256-260).
float ok_e4m3_decode(uint8_t code) {
    const int s = code >> 7;
    const int e = (code >> 3) & 0xf;
    const int m = code & 0x7;
    float v;
    if (e == 15 && m == 7) return std::nanf("");
    if (e == 0)
        v = std::ldexp(float(m), -9);
    else
        v = std::ldexp(float(8 + m), e - 10);
    return s ? -v : v;
}

uint8_t ok_e4m3_encode(float x) {
    if (std::isnan(x)) return 0x7f;
    const uint8_t sign = std::signbit(x) ? 0x80 : 0x00;
    float a = std::fabs(x);
    if (a >= 448.0f) return uint8_t(sign | 0x7e);  // callers clamp first; saturate anyway
    if (a < 0.015625f) {                             // below min normal 2^-6
        const float n = std::nearbyint(a * 512.0f);  // units of 2^-9, ties to even
        return uint8_t(sign | uint8_t(n));           // n == 8 encodes 2^-6 (e=1, m=0)
    }
    int E = std::ilogb(a);                     // -6 .. 8
    const float frac = std::ldexp(a, -E);      // [1, 2)
    int n = int(std::nearbyint((frac - 1.0f) * 8.0f));
    if (n == 8) {
        n = 0;
        E += 1;
    }
    return uint8_t(sign | uint8_t(((E + 7) << 3) | n));
}

void ok_fp8_quantize_f16(const uint16_t* src, uint8_t* dst, size_t n, float scale) {
    for (size_t i = 0; i < n; ++i) {
        float v = ok_f16_to_f32(src[i]) / scale;
        v = std::fmin(std::fmax(v, -448.0f), 448.0f);
        dst[i] = ok_e4m3_encode(v);
    }
}

// ---- a7: paged gather / attention ----------------------------------------
// Logical token t of a sequence lives in block block_table[t / block_size] at
// row t % block_size (src/experimental/server_arch/paged_kv_manager.h:56-76).
void ok_paged_gather(const void* slab, const int32_t* block_table, int seq_len, int block_size,
                     int kv_dim, int elem_bytes, void* dst) {
    const size_t row_bytes = size_t(kv_dim) * elem_bytes;
    const uint8_t* src = static_cast<const uint8_t*>(slab);
    uint8_t* out = static_cast<uint8_t*>(dst);
    for (int t = 0; t < seq_len; ++t) {
        const int64_t phys = int64_t(block_table[t / block_size]) * block_size + t % block_size;
        std::memcpy(out + size_t(t) * row_bytes, src + size_t(phys) * row_bytes, row_bytes);
    }
}

void ok_paged_attention_f16(const uint16_t* q, const uint16_t* k_slab, const uint16_t* v_slab,
                            const int32_t* block_table, int seq_len, int block_size,
                            uint16_t* out, int head_dim, int n_q_heads, int n_kv_heads) {
    const int kv_dim = n_kv_heads * head_dim;
    std::vector<uint16_t> k(size_t(seq_len) * kv_dim), v(size_t(seq_len) * kv_dim);
    ok_paged_gather(k_slab, block_table, seq_len, block_size, kv_dim, 2, k.data());
    ok_paged_gather(v_slab, block_table, seq_len, block_size, kv_dim, 2, v.data());
    ok_cached_attention(q, k.data(), v.data(), out, seq_len, head_dim, n_q_heads, n_kv_heads);
}

void ok_paged_attention_fp8(const uint16_t* q, const uint8_t* k_slab, const uint8_t* v_slab,
                            const float* k_scales, const float* v_scales,
                            const int32_t* block_table, int seq_len, int block_size,
                            uint16_t* out, int head_dim, int n_q_heads, int n_kv_heads) {
    const int kv_dim = n_kv_heads * head_dim;
    std::vector<uint8_t> k(size_t(seq_len) * kv_dim), v(size_t(seq_len) * kv_dim);
    ok_paged_gather(k_slab, block_table, seq_len, block_size, kv_dim, 1, k.data());
    ok_paged_gather(v_slab, block_table, seq_len, block_size, kv_dim, 1, v.data());
    float lut[256];
    for (int c = 0; c < 256; ++c) lut[c] = ok_e4m3_decode(uint8_t(c));
    std::vector<float> red, scores;
    for (int h = 0; h < n_q_heads; ++h) {
        const int kv_h = h * n_kv_heads / n_q_heads;
        const float ks = k_scales[kv_h], vs = v_scales[kv_h];
        const uint8_t* kb = k.data() + size_t(kv_h) * head_dim;
        const uint8_t* vb = v.data() + size_t(kv_h) * head_dim;
        auto kf = [&](int t, int d) { return lut[kb[size_t(t) * kv_dim + d]] * ks; };
        auto vf = [&](int t, int d) { return lut[vb[size_t(t) * kv_dim + d]] * vs; };
        attention_head_f32(q + size_t(h) * head_dim, seq_len, head_dim, kf, vf,
                           out + size_t(h) * head_dim, red, scores);
    }
}

void ok_paged_write_f16(const uint16_t* k_row, const uint16_t* v_row, uint16_t* k_slab,
                        uint16_t* v_slab, int64_t slot, int kv_dim) {
    std::memcpy(k_slab + size_t(slot) * kv_dim, k_row, size_t(kv_dim) * 2);
    std::memcpy(v_slab + size_t(slot) * kv_dim, v_row, size_t(kv_dim) * 2);
}

void ok_paged_write_fp8(const uint16_t* k_row, const uint16_t* v_row, uint8_t* k_slab,
                        uint8_t* v_slab, int64_t slot, int kv_dim, int head_dim,
                        const float* k_scales, const float* v_scales) {
    for (int d = 0; d < kv_dim; ++d) {
        const int h = d / head_dim;
        ok_fp8_quantize_f16(k_row + d, k_slab + size_t(slot) * kv_dim + d, 1, k_scales[h]);
        ok_fp8_quantize_f16(v_row + d, v_slab + size_t(slot) * kv_dim + d, 1, v_scales[h]);
    }
}


// ---------------------------------------------------------------------------
// W8A16 GEMV (src/kernel/qkv_gemm.cu:32-110, launched with BLOCK_DIM = 256,
// one block per output row, qkv_gemm.cu:136-151).
// Thread t of 256 accumulates elements k = 4t + 1024 j + v (v < 4), each term
// as (w * s) * x added with one rounding (nvcc contracts the multiply-add into
// an FMA by default): qkv_gemm.cu:63-90. Then each 32-thread warp reduces with
// shuffle-down offsets 16, 8, 4, 2, 1 (qkv_gemm.cu:94-96) and thread 0 adds the
// 8 warp sums in order (qkv_gemm.cu:104-109). The reference indexes scales by
// k / 128 whatever group_size says (qkv_gemm.cu:74); this restatement uses
// k / group_size, which is the same for the 128 every caller passes.
// ---------------------------------------------------------------------------
void ok_w8a16_gemv(const uint8_t* w, const uint16_t* x, const uint16_t* scales, uint16_t* y,
                   int n, int k, int group_size) {
    float lut[256];
    for (int c = 0; c < 256; ++c) lut[c] = ok_e4m3_decode(uint8_t(c));
    const int groups = k / group_size;
    std::vector<float> xf(k);
    for (int i = 0; i < k; ++i) xf[i] = ok_f16_to_f32(x[i]);
    float sum[256];
    for (int row = 0; row < n; ++row) {
        const uint8_t* wr = w + size_t(row) * k;
        const uint16_t* sr = scales + size_t(row) * groups;
        for (int t = 0; t < 256; ++t) {
            float acc = 0.0f;
            for (int kv = 4 * t; kv < k; kv += 1024) {
                const float s = ok_f16_to_f32(sr[kv / group_size]);
                for (int v = 0; v < 4; ++v) {
                    const float ws = lut[wr[kv + v]] * s;
                    acc = std::fma(ws, xf[kv + v], acc);
                }
            }
            sum[t] = acc;
        }
        float warp[8];
        for (int wi = 0; wi < 8; ++wi) {
            float* l = sum + 32 * wi;
            for (int off = 16; off > 0; off >>= 1)
                for (int i = 0; i < off; ++i) l[i] = l[i] + l[i + off];
            warp[wi] = l[0];
        }
        float total = 0.0f;
        for (int wi = 0; wi < 8; ++wi) total = total + warp[wi];
        y[row] = ok_f32_to_f16(total);
    }
}

void ok_w8a16_gemv_f64(const uint8_t* w, const uint16_t* x, const uint16_t* scales, double* y,
                       int n, int k, int group_size) {
    const int groups = k / group_size;
    for (int row = 0; row < n; ++row) {
        double acc = 0.0;
        for (int i = 0; i < k; ++i)
            acc += double(ok_e4m3_decode(w[size_t(row) * k + i])) *
                   double(ok_f16_to_f32(scales[size_t(row) * groups + i / group_size])) *
                   double(ok_f16_to_f32(x[i]));
        y[row] = acc;
    }
}
