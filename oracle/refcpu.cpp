// refcpu — CPU restatement of MobileFineTuner's attention composite.
//
// TEST INFRASTRUCTURE ONLY: the parity oracle and the CPU baseline.  Nothing
// in the product (libmft_attn.so, the finetune_ops adapter) links this file.
//
// Build: oracle/Makefile (g++ -O2 -std=c++17 -ffp-contract=off, no -march),
// the same flags the reference build uses, so that each float operation below
// rounds exactly as the reference's does.
//
// Pinning (what checks this file): tests/test_oracle.py compares it bit for
// bit with the reference compiled from its own sources (oracle/_ref) and with
// the golden fixtures in tests/golden/, and against the fp64 brute force and
// closed-form invariants (softmax rows sum to 1, O_0 = V_0 under the causal
// mask, sum_keys dV = sum_queries dO, GQA group sums).
#include "refcpu.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <vector>

namespace {

uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    uint64_t z = x;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// C[M,N] = A[M,K] * B[K,N], all row-major.  Every C[i][j] starts at 0.0f and
// accumulates a[i][k]*b[k][j] for k = 0..K-1 in increasing order, one rounding
// for the product and one for the add: the arithmetic of the reference's
// matmul_fallback_nn (core/ops.cpp:61-84).  The k-blocking only changes the
// memory traversal, never the order of additions into one C element.
void mm_nn(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K) {
    std::fill(C, C + M * N, 0.0f);
    constexpr int64_t KB = 32;
    for (int64_t k0 = 0; k0 < K; k0 += KB) {
        const int64_t k1 = std::min(K, k0 + KB);
        for (int64_t i = 0; i < M; ++i) {
            float* c = C + i * N;
            const float* a = A + i * K;
            for (int64_t kk = k0; kk < k1; ++kk) {
                const float av = a[kk];
                const float* b = B + kk * N;
                for (int64_t j = 0; j < N; ++j) c[j] += av * b[j];
            }
        }
    }
}

// Materialised 2-D transpose, as ops::transpose does for the last two dims
// (core/ops.cpp:990-1072).  Pure data movement.
void transpose2d(const float* src, float* dst, int64_t R, int64_t C) {
    for (int64_t r = 0; r < R; ++r)
        for (int64_t c = 0; c < C; ++c) dst[c * R + r] = src[r * C + c];
}

}  // namespace

extern "C" {

double orc_uniform(uint64_t seed, uint32_t stream, uint64_t counter) {
    const uint64_t z = splitmix64(seed ^ (static_cast<uint64_t>(stream) << 32) ^ counter);
    return (static_cast<double>(z >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}

void orc_fill_normal(float* x, int64_t n, uint64_t seed, uint32_t stream, float sigma) {
    const double two_pi = 6.283185307179586476925286766559;
    for (int64_t i = 0; i < n; i += 2) {
        const double u1 = orc_uniform(seed, stream, static_cast<uint64_t>(i));
        const double u2 = orc_uniform(seed, stream, static_cast<uint64_t>(i + 1));
        const double rad = std::sqrt(-2.0 * std::log(u1));
        x[i] = static_cast<float>(sigma * (rad * std::cos(two_pi * u2)));
        if (i + 1 < n) x[i + 1] = static_cast<float>(sigma * (rad * std::sin(two_pi * u2)));
    }
}

void orc_fill_mod(float* x, int64_t n, float a, int m, int o) {
    // Same expression as the reference tests: a * ((i % m) - o), the integer
    // part computed first and converted once.
    for (int64_t i = 0; i < n; ++i) x[i] = a * static_cast<float>((i % m) - o);
}

void orc_stress_rows(float* k, int64_t B, int64_t Hkv, int64_t S, int64_t D,
                     int64_t count, float factor, uint64_t seed) {
    std::vector<int64_t> perm(static_cast<size_t>(S));
    for (int64_t b = 0; b < B; ++b) {
        for (int64_t h = 0; h < Hkv; ++h) {
            for (int64_t s = 0; s < S; ++s) perm[s] = s;
            const uint64_t base = static_cast<uint64_t>((b * Hkv + h) * S);
            for (int64_t i = 0; i < count && i < S; ++i) {
                const double u = orc_uniform(seed, 4u, base + static_cast<uint64_t>(i));
                int64_t j = i + static_cast<int64_t>(u * static_cast<double>(S - i));
                if (j >= S) j = S - 1;
                std::swap(perm[i], perm[j]);
                float* row = k + ((b * Hkv + h) * S + perm[i]) * D;
                for (int64_t d = 0; d < D; ++d) row[d] *= factor;
            }
        }
    }
}

uint16_t orc_f32_to_bf16_bits(float x) {
    // Round-to-nearest-even by adding 0x7FFF + lsb, then truncating
    // (core/dtype.h:114-121).
    uint32_t bits;
    std::memcpy(&bits, &x, sizeof(bits));
    const uint32_t lsb = (bits >> 16) & 1u;
    bits += 0x7FFFu + lsb;
    return static_cast<uint16_t>(bits >> 16);
}

float orc_bf16_bits_to_f32(uint16_t b) {
    const uint32_t bits = static_cast<uint32_t>(b) << 16;
    float f;
    std::memcpy(&f, &bits, sizeof(f));
    return f;
}

void orc_round_bf16(float* x, int64_t n) {
    for (int64_t i = 0; i < n; ++i) x[i] = orc_bf16_bits_to_f32(orc_f32_to_bf16_bits(x[i]));
}

void orc_to_bf16_bits(const float* x, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_f32_to_bf16_bits(x[i]);
}

void orc_from_bf16_bits(const uint16_t* b, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_bf16_bits_to_f32(b[i]);
}

int orc_attn_composite(const float* q, const float* k, const float* v, const float* dO,
                       int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D,
                       float scale, int causal,
                       float* o, float* lse, float* dq, float* dk, float* dv) {
    return orc_attn_composite_masked(q, k, v, dO, B, Hq, Hkv, S, D, scale, causal, nullptr, nullptr, o, lse, dq,
                                     dk, dv);
}

int orc_attn_composite_masked(const float* q, const float* k, const float* v, const float* dO,
                              int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D,
                              float scale, int causal, const float* base_mask, const float* pad_mask,
                              float* o, float* lse, float* dq, float* dk, float* dv) {
    // The [S,S] base mask replaces the causal mask; the [B,1,1,S] padding
    // mask is added after it (graph/gemma_model.cpp:494-499).
    const int64_t sbase[4] = {0, 0, S, 1}, spad[4] = {S, 0, 0, 1};
    return orc_attn_composite_masks(q, k, v, dO, B, Hq, Hkv, S, D, scale, base_mask ? 0 : (causal ? 2 : 0),
                                    base_mask, sbase, pad_mask, spad, o, lse, nullptr, dq, dk, dv);
}

int orc_attn_composite_masks(const float* q, const float* k, const float* v, const float* dO,
                             int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D,
                             float scale, int mode, const float* m0, const int64_t* s0,
                             const float* m1, const int64_t* s1,
                             float* o, float* lse, float* lse2, float* dq, float* dk, float* dv) {
    if (!q || !k || !v || B <= 0 || Hq <= 0 || Hkv <= 0 || S <= 0 || D <= 0) return -1;
    if (mode < 0 || mode > 2 || (m0 && !s0) || (m1 && !s1)) return -1;
    if (Hq % Hkv != 0) return -1;
    const int64_t r = Hq / Hkv;
    const int64_t SS = S * S, SD = S * D;
    const bool want_bwd = dO != nullptr && (dq || dk || dv);

    std::vector<float> kt(SD), sc(SS), p(SS), out(SD);
    std::vector<float> vt, dp, pt, dmm, qt, dvr, dkt;
    if (want_bwd) {
        vt.resize(SD); dp.resize(SS); pt.resize(SS); dmm.resize(SS);
        qt.resize(SD); dvr.resize(SD); dkt.resize(SD);
    }
    if (dk) std::fill(dk, dk + B * Hkv * SD, 0.0f);
    if (dv) std::fill(dv, dv + B * Hkv * SD, 0.0f);

    for (int64_t b = 0; b < B; ++b) {
        for (int64_t h = 0; h < Hq; ++h) {
            const int64_t hk = h / r;  // repeat_kv_heads: out_head = kv_h * r + rep
            const float* Q = q + (b * Hq + h) * SD;
            const float* K = k + (b * Hkv + hk) * SD;
            const float* V = v + (b * Hkv + hk) * SD;

            // scores = mul(matmul(q, transpose(k, 2, 3)), scale) [+ causal mask]
            transpose2d(K, kt.data(), S, D);
            mm_nn(Q, kt.data(), sc.data(), S, S, D);
            // The causal rule of the mode, then the additive masks, one float
            // add each as the reference graphs apply them
            // (graph/gemma_model.cpp:494-499: the [S,S] base mask, e.g.
            // build_sliding_mask :272-285, then the [B,1,1,S] padding mask
            // build_padding_mask :287-321).
            for (int64_t i = 0; i < S; ++i) {
                for (int64_t j = 0; j < S; ++j) {
                    float x = sc[i * S + j] * scale;
                    if (mode == 1 && j > i) x = -1e10f;
                    if (mode == 2) x = x + (j > i ? -1e10f : 0.0f);
                    if (m0) x = x + m0[b * s0[0] + h * s0[1] + i * s0[2] + j * s0[3]];
                    if (m1) x = x + m1[b * s1[0] + h * s1[1] + i * s1[2] + j * s1[3]];
                    sc[i * S + j] = x;
                }
            }
            // softmax over the last dim: float max, exp, sequential float sum, divide.
            for (int64_t i = 0; i < S; ++i) {
                const float* row = sc.data() + i * S;
                float* pr = p.data() + i * S;
                const float mx = *std::max_element(row, row + S);
                float sum = 0.0f;
                for (int64_t j = 0; j < S; ++j) {
                    pr[j] = std::exp(row[j] - mx);
                    sum += pr[j];
                }
                for (int64_t j = 0; j < S; ++j) pr[j] /= sum;
                if (lse) {
                    // Not a reference output: the per-row log-sum-exp implied by
                    // the same max and sum, for checking the kernel's saved LSE.
                    lse[(b * Hq + h) * S + i] =
                        static_cast<float>(static_cast<double>(mx) + std::log(static_cast<double>(sum)));
                }
                if (lse2) {  // the same as (row max, ln sum)
                    lse2[2 * ((b * Hq + h) * S + i)] = mx;
                    lse2[2 * ((b * Hq + h) * S + i) + 1] = static_cast<float>(std::log(static_cast<double>(sum)));
                }
            }
            // context = matmul(probs, v)
            mm_nn(p.data(), V, out.data(), S, D, S);
            if (o) std::memcpy(o + (b * Hq + h) * SD, out.data(), sizeof(float) * SD);

            if (!want_bwd) continue;
            const float* G = dO + (b * Hq + h) * SD;
            // MatmulBackward(probs, v): dP = G v^T, dV = P^T G.
            transpose2d(V, vt.data(), S, D);
            mm_nn(G, vt.data(), dp.data(), S, S, D);
            transpose2d(p.data(), pt.data(), S, S);
            mm_nn(pt.data(), G, dvr.data(), S, D, S);
            // SoftmaxBackward: s = sum_j go*y in double, gx = y * (go - (float)s).
            // AddBackward passes the gradient through; ScaleBackward multiplies.
            for (int64_t i = 0; i < S; ++i) {
                const float* y = p.data() + i * S;
                const float* go = dp.data() + i * S;
                double s = 0.0;
                for (int64_t j = 0; j < S; ++j)
                    s += static_cast<double>(go[j]) * static_cast<double>(y[j]);
                const float sf = static_cast<float>(s);
                for (int64_t j = 0; j < S; ++j) {
                    const float gx = y[j] * (go[j] - sf);
                    dmm[i * S + j] = gx * scale;
                }
            }
            // MatmulBackward(q, k^T): dq = dMM (k^T)^T = dMM k, dk^T = q^T dMM.
            if (dq) mm_nn(dmm.data(), K, dq + (b * Hq + h) * SD, S, D, S);
            if (dk) {
                transpose2d(Q, qt.data(), S, D);
                mm_nn(qt.data(), dmm.data(), dkt.data(), D, S, S);
                float* dst = dk + (b * Hkv + hk) * SD;
                // TransposeBackward, then RepeatKVHeadsBackward's float += in rep order.
                for (int64_t j = 0; j < S; ++j)
                    for (int64_t d = 0; d < D; ++d) dst[j * D + d] += dkt[d * S + j];
            }
            if (dv) {
                float* dst = dv + (b * Hkv + hk) * SD;
                for (int64_t i = 0; i < SD; ++i) dst[i] += dvr[i];
            }
        }
    }
    return 0;
}

int orc_attn_streaming(const float* q, const float* k, const float* v,
                       int64_t B, int64_t H, int64_t S, int64_t D,
                       float scale, int causal, float* o) {
    return orc_attn_streaming_mask(q, k, v, B, H, S, D, scale, causal, nullptr, o);
}

int orc_attn_streaming_mask(const float* q, const float* k, const float* v,
                            int64_t B, int64_t H, int64_t S, int64_t D,
                            float scale, int causal, const float* mask, float* o) {
    if (!q || !k || !v || !o || B <= 0 || H <= 0 || S <= 0 || D <= 0) return -1;
    std::vector<float> scores(static_cast<size_t>(S));
    for (int64_t bh = 0; bh < B * H; ++bh) {
        const float* Q = q + bh * S * D;
        const float* K = k + bh * S * D;
        const float* V = v + bh * S * D;
        float* O = o + bh * S * D;
        for (int64_t i = 0; i < S; ++i) {
            const float* qr = Q + i * D;
            float mx = -INFINITY;
            for (int64_t j = 0; j < S; ++j) {
                const float* kr = K + j * D;
                float dot = 0.0f;
                for (int64_t d = 0; d < D; ++d) dot += qr[d] * kr[d];
                float s = dot * scale;
                if (causal && j > i) s = -1e10f;
                if (mask) s += mask[i * S + j];
                scores[j] = s;
                mx = std::max(mx, s);
            }
            float* orow = O + i * D;
            std::fill(orow, orow + D, 0.0f);
            double sum_exp = 0.0;
            for (int64_t j = 0; j < S; ++j) sum_exp += std::exp(scores[j] - mx);
            const float inv = 1.0f / static_cast<float>(sum_exp);
            for (int64_t j = 0; j < S; ++j) {
                const float w = std::exp(scores[j] - mx) * inv;
                const float* vr = V + j * D;
                for (int64_t d = 0; d < D; ++d) orow[d] += w * vr[d];
            }
        }
    }
    return 0;
}

int orc_attn_f64(const float* q, const float* k, const float* v, const float* dO,
                 int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D,
                 double scale, int causal,
                 double* o, double* lse, double* dq, double* dk, double* dv) {
    if (!q || !k || !v || B <= 0 || Hq <= 0 || Hkv <= 0 || S <= 0 || D <= 0) return -1;
    if (Hq % Hkv != 0) return -1;
    const int64_t r = Hq / Hkv, SD = S * D;
    std::vector<double> P(S * S), dP(S * S);
    if (dk) std::fill(dk, dk + B * Hkv * SD, 0.0);
    if (dv) std::fill(dv, dv + B * Hkv * SD, 0.0);
    for (int64_t b = 0; b < B; ++b) {
        for (int64_t h = 0; h < Hq; ++h) {
            const int64_t hk = h / r;
            const float* Q = q + (b * Hq + h) * SD;
            const float* K = k + (b * Hkv + hk) * SD;
            const float* V = v + (b * Hkv + hk) * SD;
            for (int64_t i = 0; i < S; ++i) {
                const int64_t jn = causal ? i + 1 : S;
                double mx = -INFINITY;
                for (int64_t j = 0; j < jn; ++j) {
                    double s = 0.0;
                    for (int64_t d = 0; d < D; ++d) s += double(Q[i * D + d]) * double(K[j * D + d]);
                    P[i * S + j] = s * scale;
                    mx = std::max(mx, P[i * S + j]);
                }
                double sum = 0.0;
                for (int64_t j = 0; j < jn; ++j) {
                    P[i * S + j] = std::exp(P[i * S + j] - mx);
                    sum += P[i * S + j];
                }
                for (int64_t j = 0; j < jn; ++j) P[i * S + j] /= sum;
                for (int64_t j = jn; j < S; ++j) P[i * S + j] = 0.0;
                if (lse) lse[(b * Hq + h) * S + i] = mx + std::log(sum);
                if (o) {
                    for (int64_t d = 0; d < D; ++d) {
                        double acc = 0.0;
                        for (int64_t j = 0; j < jn; ++j) acc += P[i * S + j] * double(V[j * D + d]);
                        o[(b * Hq + h) * SD + i * D + d] = acc;
                    }
                }
            }
            if (!dO) continue;
            const float* G = dO + (b * Hq + h) * SD;
            for (int64_t i = 0; i < S; ++i) {
                double delta = 0.0;
                for (int64_t j = 0; j < S; ++j) {
                    double s = 0.0;
                    for (int64_t d = 0; d < D; ++d) s += double(G[i * D + d]) * double(V[j * D + d]);
                    dP[i * S + j] = s;
                    delta += s * P[i * S + j];
                }
                for (int64_t j = 0; j < S; ++j) dP[i * S + j] = P[i * S + j] * (dP[i * S + j] - delta);
            }
            for (int64_t i = 0; i < S; ++i) {
                for (int64_t d = 0; d < D; ++d) {
                    if (dq) {
                        double acc = 0.0;
                        for (int64_t j = 0; j < S; ++j) acc += dP[i * S + j] * double(K[j * D + d]);
                        dq[(b * Hq + h) * SD + i * D + d] = acc * scale;
                    }
                }
            }
            for (int64_t j = 0; j < S; ++j) {
                for (int64_t d = 0; d < D; ++d) {
                    double ak = 0.0, av = 0.0;
                    for (int64_t i = 0; i < S; ++i) {
                        ak += dP[i * S + j] * double(Q[i * D + d]);
                        av += P[i * S + j] * double(G[i * D + d]);
                    }
                    if (dk) dk[(b * Hkv + hk) * SD + j * D + d] += ak * scale;
                    if (dv) dv[(b * Hkv + hk) * SD + j * D + d] += av;
                }
            }
        }
    }
    return 0;
}

void orc_repeat_kv(const float* kv, float* out, int64_t B, int64_t Hkv, int64_t S,
                   int64_t D, int64_t r) {
    const int64_t SD = S * D;
    for (int64_t b = 0; b < B; ++b)
        for (int64_t h = 0; h < Hkv; ++h)
            for (int64_t rep = 0; rep < r; ++rep)
                std::memcpy(out + (b * Hkv * r + h * r + rep) * SD, kv + (b * Hkv + h) * SD,
                            sizeof(float) * SD);
}

void orc_repeat_kv_backward(const float* g, float* dkv, int64_t B, int64_t Hkv,
                            int64_t S, int64_t D, int64_t r) {
    const int64_t SD = S * D;
    std::fill(dkv, dkv + B * Hkv * SD, 0.0f);
    for (int64_t b = 0; b < B; ++b)
        for (int64_t h = 0; h < Hkv; ++h)
            for (int64_t rep = 0; rep < r; ++rep) {
                const float* src = g + (b * Hkv * r + h * r + rep) * SD;
                float* dst = dkv + (b * Hkv + h) * SD;
                for (int64_t i = 0; i < SD; ++i) dst[i] += src[i];
            }
}

// ---- q/k prologue ----

namespace {

// RoPE of one row in place (core/ops.cpp:2363-2389): rotate-half pairs.
void rope_row(float* r, int64_t pos, int64_t D, float theta) {
    const int64_t half = D / 2;
    for (int64_t d = 0; d < half; ++d) {
        float freq = 1.0f / std::pow(theta, 2.0f * d / D);
        float angle = pos * freq;
        float c = std::cos(angle);
        float s = std::sin(angle);
        float x1 = r[d];
        float x2 = r[half + d];
        r[d] = x1 * c - x2 * s;
        r[half + d] = x1 * s + x2 * c;
    }
}

}  // namespace

void orc_prologue_fwd(const float* x, const float* w, int64_t B, int64_t H, int64_t S, int64_t D,
                      int norm, float eps, float theta, float* y) {
    const int64_t rows = B * H * S;
    for (int64_t r = 0; r < rows; ++r) {
        const float* xr = x + r * D;
        float* yr = y + r * D;
        if (norm == 0) {
            std::memcpy(yr, xr, sizeof(float) * D);
        } else {
            double ss = 0.0;
            for (int64_t i = 0; i < D; ++i) ss += static_cast<double>(xr[i]) * static_cast<double>(xr[i]);
            if (norm == 1) {
                float rms = static_cast<float>(std::sqrt(ss / static_cast<double>(D) + static_cast<double>(eps)));
                for (int64_t i = 0; i < D; ++i) {
                    float scale = 1.0f + w[i];
                    yr[i] = (xr[i] / rms) * scale;
                }
            } else {
                float inv = static_cast<float>(1.0 / std::sqrt(ss / static_cast<double>(D) + static_cast<double>(eps)));
                for (int64_t i = 0; i < D; ++i) yr[i] = xr[i] * inv * w[i];
            }
        }
        if (theta > 0.f) rope_row(yr, r % S, D, theta);
    }
}

void orc_prologue_bwd(const float* x, const float* w, const float* dy, int64_t B, int64_t H, int64_t S,
                      int64_t D, int norm, float eps, float theta, float* dx, float* dw) {
    const int64_t rows = B * H * S, half = D / 2;
    std::vector<float> g(D);
    if (dw) std::fill(dw, dw + D, 0.0f);
    for (int64_t r = 0; r < rows; ++r) {
        const float* gy = dy + r * D;
        if (theta > 0.f) {
            const int64_t pos = r % S;
            for (int64_t d = 0; d < half; ++d) {
                float freq = 1.0f / std::pow(theta, 2.0f * static_cast<float>(d) / static_cast<float>(D));
                float angle = static_cast<float>(pos) * freq;
                float c = std::cos(angle);
                float s = std::sin(angle);
                float g1p = gy[d];
                float g2p = gy[half + d];
                g[d] = g1p * c + g2p * s;
                g[half + d] = -g1p * s + g2p * c;
            }
        } else {
            std::memcpy(g.data(), gy, sizeof(float) * D);
        }
        float* gx = dx + r * D;
        if (norm == 0) {
            std::memcpy(gx, g.data(), sizeof(float) * D);
            continue;
        }
        const float* xb = x + r * D;
        double sqsum = 0.0;
        for (int64_t i = 0; i < D; ++i) sqsum += static_cast<double>(xb[i]) * static_cast<double>(xb[i]);
        double inv_rms = 1.0 / std::sqrt(sqsum / static_cast<double>(D) + static_cast<double>(eps));
        auto w_eff = [&](int64_t i) {
            return norm == 1 ? 1.0 + static_cast<double>(w[i]) : static_cast<double>(w[i]);
        };
        double dot = 0.0;
        for (int64_t i = 0; i < D; ++i) dot += static_cast<double>(g[i]) * w_eff(i) * static_cast<double>(xb[i]);
        double coeff = (inv_rms * inv_rms * inv_rms) / static_cast<double>(D);
        for (int64_t i = 0; i < D; ++i) {
            double term1 = static_cast<double>(g[i]) * w_eff(i) * inv_rms;
            double term2 = static_cast<double>(xb[i]) * coeff * dot;
            gx[i] = static_cast<float>(term1 - term2);
            if (dw) dw[i] += static_cast<float>(static_cast<double>(g[i]) * static_cast<double>(xb[i]) * inv_rms);
        }
    }
}

// ---- LM cross-entropy ----

int orc_lm_ce(const float* logits, const int32_t* labels, int64_t B, int64_t S, int64_t V, int ignore_index,
              int reduction, const float* grad_out, float* loss, float* grad_logits) {
    // forward (core/lm_loss.cpp:291-313, 318-334)
    double loss_sum = 0.0;
    int64_t valid_cnt = 0;
    for (int64_t b = 0; b < B; ++b)
        for (int64_t s = 0; s < S; ++s) {
            if (reduction == 2) loss[b * S + s] = 0.0f;
            if (s + 1 >= S) continue;
            int32_t cls = labels[b * S + (s + 1)];
            if (cls == ignore_index) continue;
            if (cls < 0 || cls >= V) return -1;
            const float* row = logits + (b * S + s) * V;
            float max_val = -std::numeric_limits<float>::infinity();
            for (int64_t v = 0; v < V; ++v) max_val = std::max(max_val, row[v]);
            double denom = 0.0;
            for (int64_t v = 0; v < V; ++v) denom += std::exp(row[v] - max_val);
            double log_sum_exp = max_val + std::log(denom);
            loss_sum += (log_sum_exp - row[cls]);
            valid_cnt++;
            if (reduction == 2) loss[b * S + s] = static_cast<float>(log_sum_exp - row[cls]);
        }
    if (reduction == 1) loss[0] = static_cast<float>(loss_sum);
    if (reduction == 0)
        loss[0] = valid_cnt > 0 ? static_cast<float>(loss_sum / static_cast<double>(valid_cnt))
                                : std::numeric_limits<float>::quiet_NaN();
    if (!grad_out || !grad_logits) return 0;
    // backward (core/lm_loss.cpp:85-158)
    std::fill(grad_logits, grad_logits + B * S * V, 0.0f);
    float scale_base = 1.0f;
    if (reduction == 0) scale_base = (valid_cnt > 0) ? (1.0f / static_cast<float>(valid_cnt)) : 0.0f;
    for (int64_t b = 0; b < B; ++b)
        for (int64_t s = 0; s + 1 < S; ++s) {
            int32_t y = labels[b * S + (s + 1)];
            if (y == ignore_index) continue;
            const float* logit_row = logits + (b * S + s) * V;
            float max_val = -std::numeric_limits<float>::infinity();
            for (int64_t v = 0; v < V; ++v) max_val = std::max(max_val, logit_row[v]);
            float denom = 0.0f;
            for (int64_t v = 0; v < V; ++v) denom += std::exp(logit_row[v] - max_val);
            float inv_denom = 1.0f / denom;
            float outer = reduction == 2 ? grad_out[b * S + s] : grad_out[0];
            float coeff = outer * scale_base;
            float* grad_row = grad_logits + (b * S + s) * V;
            for (int64_t v = 0; v < V; ++v) {
                float p = std::exp(logit_row[v] - max_val) * inv_denom;
                float g = p;
                if (v == y) g -= 1.0f;
                grad_row[v] = g * coeff;
            }
        }
    return 0;
}

int orc_selected_ce(const float* hidden, const float* weight, const int32_t* labels, int64_t B, int64_t S,
                    int64_t H, int64_t V, int ignore_index, int reduction, float grad_out, float* loss,
                    float* grad_hidden, float* grad_weight) {
    struct Item {
        int64_t b, s;
        int32_t cls;
    };
    std::vector<Item> valid;  // core/lm_loss.cpp:28-47
    for (int64_t b = 0; b < B; ++b)
        for (int64_t s = 0; s + 1 < S; ++s) {
            int32_t cls = labels[b * S + (s + 1)];
            if (cls == ignore_index) continue;
            if (cls < 0 || cls >= V) return -1;
            valid.push_back({b, s, cls});
        }
    auto dot = [&](const float* hrow, int64_t v) {  // :63-70
        float sum = 0.0f;
        for (int64_t h = 0; h < H; ++h) sum += hrow[h] * weight[v * H + h];
        return sum;
    };
    // forward (:420-451)
    double loss_sum = 0.0;
    for (const Item& it : valid) {
        const float* hrow = hidden + (it.b * S + it.s) * H;
        float max_val = -std::numeric_limits<float>::infinity();
        float target_logit = 0.0f;
        for (int64_t v = 0; v < V; ++v) {
            const float z = dot(hrow, v);
            if (v == it.cls) target_logit = z;
            max_val = std::max(max_val, z);
        }
        double denom = 0.0;
        for (int64_t v = 0; v < V; ++v) denom += std::exp(dot(hrow, v) - max_val);
        const double log_sum_exp = max_val + std::log(denom);
        loss_sum += (log_sum_exp - target_logit);
    }
    if (reduction == 1)
        loss[0] = static_cast<float>(loss_sum);
    else
        loss[0] = valid.empty() ? std::numeric_limits<float>::quiet_NaN()
                                : static_cast<float>(loss_sum / static_cast<double>(valid.size()));
    if (!grad_hidden && !grad_weight) return 0;
    // backward (:197-262)
    if (grad_hidden) std::fill(grad_hidden, grad_hidden + B * S * H, 0.0f);
    if (grad_weight) std::fill(grad_weight, grad_weight + V * H, 0.0f);
    if (valid.empty()) return 0;
    float scale_base = 1.0f;
    if (reduction == 0) scale_base = 1.0f / static_cast<float>(valid.size());
    const float coeff = grad_out * scale_base;
    if (coeff == 0.0f) return 0;
    std::vector<float> logits(static_cast<size_t>(V));
    for (const Item& it : valid) {
        const float* hrow = hidden + (it.b * S + it.s) * H;
        float max_val = -std::numeric_limits<float>::infinity();
        for (int64_t v = 0; v < V; ++v) {
            const float z = dot(hrow, v);
            logits[static_cast<size_t>(v)] = z;
            max_val = std::max(max_val, z);
        }
        float denom = 0.0f;
        for (int64_t v = 0; v < V; ++v) denom += std::exp(logits[static_cast<size_t>(v)] - max_val);
        const float inv_denom = 1.0f / denom;
        float* ghrow = grad_hidden ? grad_hidden + (it.b * S + it.s) * H : nullptr;
        for (int64_t v = 0; v < V; ++v) {
            float p = std::exp(logits[static_cast<size_t>(v)] - max_val) * inv_denom;
            if (v == it.cls) p -= 1.0f;
            const float g = p * coeff;
            if (ghrow)
                for (int64_t h = 0; h < H; ++h) ghrow[h] += g * weight[v * H + h];
            if (grad_weight) {
                float* gwrow = grad_weight + v * H;
                for (int64_t h = 0; h < H; ++h) gwrow[h] += g * hrow[h];
            }
        }
    }
    return 0;
}


// ---- LoRA linear ----

// A_eff [in, r] and B_eff [r, cols] of slice i (materialised transposes, as
// the reference's transpose() makes them), and the offsets of the next slice.
static void lora_eff(const int64_t* m, int64_t in, const float* A, const float* B, std::vector<float>& Ae,
                     std::vector<float>& Be) {
    const int64_t r = m[0], cols = m[2];
    Ae.assign(A, A + in * r);
    Be.assign(B, B + r * cols);
    if (m[3]) transpose2d(A, Ae.data(), r, in);
    if (m[4]) transpose2d(B, Be.data(), cols, r);
}

// C[M,N] = A[M,K] . B[N,K]^T with the association of the reference's
// matmul_fallback_nt_mixed_b (core/ops.cpp:211-246), its path for a bf16
// right operand: per 64-wide block of k a fresh float sum in k order, added
// to C[i][j] block by block.
static void mm_nt_blocked64(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K) {
    std::fill(C, C + M * N, 0.0f);
    for (int64_t k0 = 0; k0 < K; k0 += 64) {
        const int64_t k1 = std::min(K, k0 + 64);
        for (int64_t i = 0; i < M; ++i)
            for (int64_t j = 0; j < N; ++j) {
                float sum = 0.0f;
                for (int64_t k = k0; k < k1; ++k) sum += A[i * K + k] * B[j * K + k];
                C[i * N + j] += sum;
            }
    }
}

void orc_lora(const float* x, const float* W, const float* bias, int64_t N, int64_t in, int64_t out, int w_transposed,
              int w_lowp, int n, const int64_t* meta, const float* scale, const float* A_all, const float* B_all,
              int all_grads, const float* dy, float* y, float* dx, float* dA_all, float* dB_all, int32_t* has_grad) {
    // Base: y = matmul(x, W_eff), W_eff = W or its transpose [in, out].
    std::vector<float> We(W, W + in * out);
    if (w_transposed) transpose2d(W, We.data(), out, in);
    mm_nn(x, We.data(), y, N, out, in);
    if (bias)
        for (int64_t i = 0; i < N; ++i)
            for (int64_t o = 0; o < out; ++o) y[i * out + o] = y[i * out + o] + bias[o];
    std::vector<float> Ae, Be, xa, delta, ds, g, tmp, tmp2;
    const float* Ap = A_all;
    const float* Bp = B_all;
    std::vector<std::vector<float>> gs(n), Aes(n);
    for (int i = 0; i < n; ++i) {
        const int64_t* m = meta + 5 * i;
        const int64_t r = m[0], col0 = m[1], cols = m[2];
        lora_eff(m, in, Ap, Bp, Ae, Be);
        xa.assign(N * r, 0.f);
        mm_nn(x, Ae.data(), xa.data(), N, r, in);
        delta.assign(N * cols, 0.f);
        mm_nn(xa.data(), Be.data(), delta.data(), N, cols, r);
        for (auto& v : delta) v = v * scale[i];
        for (int64_t t = 0; t < N; ++t)
            for (int64_t c = 0; c < cols; ++c) y[t * out + col0 + c] = y[t * out + col0 + c] + delta[t * cols + c];
        const bool grad = all_grads || (col0 == 0 && cols == out);
        if (has_grad) has_grad[i] = grad;
        if (dy && grad) {
            // d(delta2d) = mul backward: dy_slice * scale
            ds.assign(N * cols, 0.f);
            for (int64_t t = 0; t < N; ++t)
                for (int64_t c = 0; c < cols; ++c) ds[t * cols + c] = dy[t * out + col0 + c] * scale[i];
            // g = ds . B_eff^T  [N, r]
            tmp.assign(cols * r, 0.f);
            transpose2d(Be.data(), tmp.data(), r, cols);
            gs[i].assign(N * r, 0.f);
            mm_nn(ds.data(), tmp.data(), gs[i].data(), N, r, cols);
            // grad_B_eff = xa^T . ds  [r, cols]
            tmp.assign(r * N, 0.f);
            transpose2d(xa.data(), tmp.data(), N, r);
            tmp2.assign(r * cols, 0.f);
            mm_nn(tmp.data(), ds.data(), tmp2.data(), r, cols, N);
            float* dB = dB_all + (Bp - B_all);
            if (m[4]) transpose2d(tmp2.data(), dB, r, cols);
            else std::copy(tmp2.begin(), tmp2.end(), dB);
            // grad_A_eff = x^T . g  [in, r]
            tmp.assign(in * N, 0.f);
            transpose2d(x, tmp.data(), N, in);
            tmp2.assign(in * r, 0.f);
            mm_nn(tmp.data(), gs[i].data(), tmp2.data(), in, r, N);
            float* dA = dA_all + (Ap - A_all);
            if (m[3]) transpose2d(tmp2.data(), dA, in, r);
            else std::copy(tmp2.begin(), tmp2.end(), dA);
            Aes[i] = Ae;
        }
        Ap += in * r;
        Bp += r * cols;
    }
    if (!dy || !dx) return;
    // dx = dy . W_eff^T (MatmulBackward: matmul_rhs_T, core/backward_functions.cpp:98-101), then each
    // slice's g . A_eff^T added in slice order.
    if (w_lowp) {
        mm_nt_blocked64(dy, We.data(), dx, N, in, out);
    } else {
        tmp.assign(out * in, 0.f);
        transpose2d(We.data(), tmp.data(), in, out);
        mm_nn(dy, tmp.data(), dx, N, in, out);
    }
    for (int i = 0; i < n; ++i) {
        if (gs[i].empty()) continue;
        const int64_t r = meta[5 * i];
        tmp.assign(r * in, 0.f);
        transpose2d(Aes[i].data(), tmp.data(), in, r);
        tmp2.assign(N * in, 0.f);
        mm_nn(gs[i].data(), tmp.data(), tmp2.data(), N, in, r);
        for (int64_t t = 0; t < N * in; ++t) dx[t] = dx[t] + tmp2[t];
    }
}

void orc_lora_merge(float* W, int w_bf16, int64_t in, int64_t out, int n, const int64_t* meta, const float* scale,
                    const float* A_all, const float* B_all, float sign) {
    const float* Ap = A_all;
    const float* Bp = B_all;
    for (int s = 0; s < n; ++s) {
        const int64_t* m = meta + 5 * s;
        const int64_t r = m[0], col0 = m[1], cols = m[2];
        for (int64_t i = 0; i < in; ++i)
            for (int64_t o = 0; o < cols; ++o) {
                double delta = 0.0;
                for (int64_t k = 0; k < r; ++k) {
                    const float a = m[3] ? Ap[k * in + i] : Ap[i * r + k];
                    const float b = m[4] ? Bp[o * r + k] : Bp[k * cols + o];
                    delta += static_cast<double>(a) * static_cast<double>(b);
                }
                float& w = W[i * out + col0 + o];
                const float updated = w + sign * scale[s] * static_cast<float>(delta);
                w = w_bf16 ? orc_bf16_bits_to_f32(orc_f32_to_bf16_bits(updated)) : updated;
            }
        Ap += in * r;
        Bp += r * cols;
    }
}

}  // extern "C"
