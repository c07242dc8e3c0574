/*
 * TEST INFRASTRUCTURE ONLY — the CPU oracle for fracture_amd's parity tests.
 *
 * A plain-C restatement of the reference's own arithmetic for the hot path, each function
 * citing the reference file:line it follows (paths relative to the nickw409/Fracture tree).
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 * library, and only as the checker / the timed CPU baseline; the product never calls it.
 *
 * Built with -O2 -ffp-contract=off: single-precision and double-precision operations are
 * evaluated one IEEE operation at a time, in the order the Rust CPU code (which never
 * fuses) evaluates them; libm (glibc) provides exp/log/sin/cos/pow as it does for Rust.
 *
 * What pins each function (checks live in tests/test_oracle_*.py):
 *   f16/bf16 conversions ... numpy's correctly rounded float16 / round-to-nearest-even bf16
 *   add, rmsnorm, silu_mul, rope, embedding ... the reference's PyTorch fixture dumps
 *   argmax ............ fixture logits -> greedy_token, sampler unit-test vector, brute force
 *   softmax ........... closed forms (sum 1, ratios exp(xi-xj)), float64 recomputation
 *   codebook .......... Max (1960) Gaussian quantizer tables, symmetry, sqrt(2) scaling
 *   rotation .......... published SplitMix64 / xoshiro256** outputs, Q^T Q = I, Q^T G upper
 *                       triangular with the diagonal sign rule
 *   quantize/pack ..... brute force over all codes, explicit 2/4/8-bit byte layouts of the
 *                       reference kernel vs the MSB-first generalisation
 *   compress/dequant .. composition of the above + round-trip cosine thresholds
 *   attention ......... float64 softmax attention over dequantized K/V, rotation identities
 *   paged attention ... float64 softmax(QK^T/sqrt(d))V, one-position and equal-key closed forms,
 *                       page-permutation invariance
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------------------------------
 * fp16 / bf16 conversions (the `half` crate 2.7.1: IEEE round-to-nearest-even)
 * ------------------------------------------------------------------------------------- */
uint16_t o_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
    if (ax < 0x38800000u) {                                   /* half subnormal or zero */
        float af;
        memcpy(&af, &ax, 4);
        const float m = af * 16777216.0f; /* exact: times 2^24 */
        return (uint16_t)(sign | (uint32_t)nearbyintf(m));
    }
    const uint32_t mant = ax & 0x7fffffu;
    const uint32_t e = (ax >> 23) - 127u + 15u;
    uint32_t h = (e << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
}

float o_f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else {
            float f = (float)m * (1.0f / 16777216.0f); /* m * 2^-24, exact */
            memcpy(&x, &f, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e - 15u + 127u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

uint16_t o_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float o_bf16_to_f32(uint16_t b) {
    const uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

void o_f32_to_f16_array(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = o_f32_to_f16(in[i]);
}
void o_f16_to_f32_array(const uint16_t* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = o_f16_to_f32(in[i]);
}

/* dtype codes shared with the library: 0 = fp16, 1 = fp32, 2 = bf16 */
static float ld(const void* p, int64_t i, int dt) {
    if (dt == 0) return o_f16_to_f32(((const uint16_t*)p)[i]);
    if (dt == 2) return o_bf16_to_f32(((const uint16_t*)p)[i]);
    return ((const float*)p)[i];
}
static void st(void* p, int64_t i, float v, int dt) {
    if (dt == 0)
        ((uint16_t*)p)[i] = o_f32_to_f16(v);
    else if (dt == 2)
        ((uint16_t*)p)[i] = o_f32_to_bf16(v);
    else
        ((float*)p)[i] = v;
}

/* ---------------------------------------------------------------------------------------
 * Elementwise / normalisation
 * ------------------------------------------------------------------------------------- */

/* add: f16(f32(a) + f32(b)) (backends/fracture-cuda/src/tests.rs:2051-2054). */
void o_add(const void* a, const void* b, void* out, int64_t n, int dt) {
    for (int64_t i = 0; i < n; ++i) st(out, i, ld(a, i, dt) + ld(b, i, dt), dt);
}

/* RMSNorm, the CPU reference of backends/fracture-cuda/src/tests.rs:576-585:
 * mean_sq = (sum of v*v, sequential f32) / cols; rms = sqrt(mean_sq + eps);
 * out = (v / rms) * w, eps as f32 (backend.rs:152). */
void o_rmsnorm(const void* x, const void* w, float eps, void* out, int64_t rows, int64_t cols,
               int dt) {
    for (int64_t r = 0; r < rows; ++r) {
        float ss = 0.0f;
        for (int64_t j = 0; j < cols; ++j) {
            const float v = ld(x, r * cols + j, dt);
            ss += v * v;
        }
        const float mean_sq = ss / (float)cols;
        const float rms = sqrtf(mean_sq + eps);
        for (int64_t j = 0; j < cols; ++j)
            st(out, r * cols + j, (ld(x, r * cols + j, dt) / rms) * ld(w, j, dt), dt);
    }
}

/* Residual add then RMSNorm, as the engine runs them (crates/fracture-engine/src/
 * engine.rs:692-697): h = dtype(h + d) in place, out = rmsnorm(h). */
void o_add_rmsnorm(void* h, const void* d, const void* w, float eps, void* out, int64_t rows,
                   int64_t cols, int dt) {
    o_add(h, d, h, rows * cols, dt);
    o_rmsnorm(h, w, eps, out, rows, cols, dt);
}

/* silu(g) * u with silu(x) = x / (1 + exp(-x)) in f32 (tests.rs:251-255, silu_mul.cu:17-22). */
void o_silu_mul(const void* g, const void* u, void* out, int64_t n, int dt) {
    for (int64_t i = 0; i < n; ++i) {
        const float x = ld(g, i, dt);
        const float s = x / (1.0f + expf(-x));
        st(out, i, s * ld(u, i, dt), dt);
    }
}

/* RoPE inverse frequencies (backends/fracture-cuda/src/lib.rs:134-139):
 * freq[i] = 1f32 / (theta.powf(2i / hd) as f32), the power in f64. */
void o_rope_freqs(int hd, double theta, float* out) {
    for (int i = 0; i < hd / 2; ++i) {
        const double p = pow(theta, 2.0 * (double)i / (double)hd);
        out[i] = 1.0f / (float)p;
    }
}

/* Split-half RoPE in place (rope.cu:33-48; CPU form tests.rs:2469-2477):
 * angle = (float)pos * freq[d]; (x0, x1) -> (x0 c - x1 s, x0 s + x1 c). */
void o_rope(void* x, const uint32_t* pos, const float* freq, int64_t tokens, int64_t heads,
            int64_t hd, int dt) {
    const int64_t half = hd / 2;
    for (int64_t t = 0; t < tokens; ++t)
        for (int64_t h = 0; h < heads; ++h)
            for (int64_t d = 0; d < half; ++d) {
                const float angle = (float)pos[t] * freq[d];
                const float s = sinf(angle), c = cosf(angle);
                const int64_t base = (t * heads + h) * hd;
                const float x0 = ld(x, base + d, dt), x1 = ld(x, base + d + half, dt);
                const float lo = x0 * c - x1 * s;
                const float hi = x0 * s + x1 * c;
                st(x, base + d, lo, dt);
                st(x, base + d + half, hi, dt);
            }
}

/* Embedding gather (embedding.cu:21-27): rows of elem_bytes-sized elements, zeros for
 * ids >= vocab. */
void o_embedding(const void* table, const uint32_t* ids, void* out, int64_t tokens,
                 int64_t hidden, int64_t vocab, int elem_bytes) {
    const int64_t row = hidden * elem_bytes;
    for (int64_t t = 0; t < tokens; ++t) {
        if (ids[t] < (uint64_t)vocab)
            memcpy((char*)out + t * row, (const char*)table + (int64_t)ids[t] * row, (size_t)row);
        else
            memset((char*)out + t * row, 0, (size_t)row);
    }
}

/* ---------------------------------------------------------------------------------------
 * Sampler: greedy argmax and softmax (crates/fracture-generate/src/sampling.rs:31-82)
 * ------------------------------------------------------------------------------------- */

/* Returns 0 and the index, or 1 = empty, 2 = NaN in logits, 3 = Inf in logits.
 * Ties go to the last index (Iterator::max_by keeps the last of equal elements). */
int o_argmax(const float* l, int64_t n, int64_t* idx_out) {
    if (n == 0) return 1;
    for (int64_t i = 0; i < n; ++i)
        if (isnan(l[i])) return 2;
    for (int64_t i = 0; i < n; ++i)
        if (isinf(l[i])) return 3;
    int64_t best = 0;
    for (int64_t i = 1; i < n; ++i)
        if (!(l[i] < l[best])) best = i; /* >= : later equal elements win */
    *idx_out = best;
    return 0;
}

/* Softmax body for top_k = 0 (sampling.rs:69-82): scaled = l / T; m = fold(-inf, max);
 * e = exp(scaled - m); s = sequential f32 sum of e; p = e / s. */
void o_softmax(const float* l, float* p, int64_t n, float temperature) {
    float m = -INFINITY;
    for (int64_t i = 0; i < n; ++i) {
        const float v = l[i] / temperature;
        m = fmaxf(m, v);
    }
    float s = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        p[i] = expf(l[i] / temperature - m);
        s += p[i];
    }
    for (int64_t i = 0; i < n; ++i) p[i] = p[i] / s;
}

void o_softmax_rows(const float* l, float* p, int64_t rows, int64_t cols, float temperature) {
    for (int64_t r = 0; r < rows; ++r) o_softmax(l + r * cols, p + r * cols, cols, temperature);
}

int o_argmax_rows(const float* l, int64_t rows, int64_t cols, int64_t* idx, int* status) {
    int worst = 0;
    for (int64_t r = 0; r < rows; ++r) {
        idx[r] = -1;
        status[r] = o_argmax(l + r * cols, cols, &idx[r]);
        if (status[r] > worst) worst = status[r];
    }
    return worst;
}

/* ---------------------------------------------------------------------------------------
 * TurboQuant host math (crates/fracture-core/src/turboquant.rs)
 * ------------------------------------------------------------------------------------- */
static const double O_PI = 3.14159265358979323846;

/* turboquant.rs:166-168 */
static double o_pdf(double x, double sigma2) {
    return (1.0 / sqrt(2.0 * O_PI * sigma2)) * exp(-x * x / (2.0 * sigma2));
}

/* turboquant.rs:171-180; which = 0: integrand pdf(x), 1: x * pdf(x). */
static double o_simpson(int which, double sigma2, double a, double b, int n) {
    if (n % 2 == 1) n += 1;
    const double h = (b - a) / (double)n;
    double fa = o_pdf(a, sigma2), fb = o_pdf(b, sigma2);
    if (which) {
        fa = a * fa;
        fb = b * fb;
    }
    double sum = fa + fb;
    for (int i = 1; i < n; ++i) {
        const double x = a + (double)i * h;
        double fx = o_pdf(x, sigma2);
        if (which) fx = x * o_pdf(x, sigma2);
        sum += (i % 2 == 0) ? 2.0 * fx : 4.0 * fx;
    }
    return sum * h / 3.0;
}

/* LloydMaxCodebook::compute (turboquant.rs:186-250); returns the iteration count used. */
int o_lloyd_max(int dim, int bits, float* centroids, float* boundaries) {
    const int L = 1 << bits;
    const double sigma2 = 1.0 / (double)dim;
    const double sigma = sqrt(sigma2);
    const double lo = -3.5 * sigma, hi = 3.5 * sigma;
    double* c = (double*)malloc(sizeof(double) * (size_t)L);
    double* nc = (double*)malloc(sizeof(double) * (size_t)L);
    double* bd = (double*)malloc(sizeof(double) * (size_t)(L > 1 ? L - 1 : 1));
    for (int i = 0; i < L; ++i) c[i] = lo + (hi - lo) * ((double)i + 0.5) / (double)L;
    int it;
    for (it = 0; it < 200; ++it) {
        for (int i = 0; i + 1 < L; ++i) bd[i] = (c[i] + c[i + 1]) / 2.0;
        const double elo = lo * 3.0, ehi = hi * 3.0;
        double shift = 0.0;
        for (int i = 0; i < L; ++i) {
            const double a = i == 0 ? elo : bd[i - 1];
            const double b = i == L - 1 ? ehi : bd[i];
            const double num = o_simpson(1, sigma2, a, b, 500);
            const double den = o_simpson(0, sigma2, a, b, 500);
            nc[i] = fabs(den) > 1e-15 ? num / den : c[i];
            const double dlt = fabs(nc[i] - c[i]);
            if (dlt > shift) shift = dlt;
        }
        double* t = c;
        c = nc;
        nc = t;
        if (shift < 1e-10) {
            ++it;
            break;
        }
    }
    for (int i = 0; i < L; ++i) centroids[i] = (float)c[i];
    if (boundaries)
        for (int i = 0; i + 1 < L; ++i) boundaries[i] = (float)((c[i] + c[i + 1]) / 2.0);
    free(c);
    free(nc);
    free(bd);
    return it;
}

/* SplitMix64 -> xoshiro256** (turboquant.rs:349-385) */
typedef struct {
    uint64_t s[4];
} o_rng;

static uint64_t o_rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

void o_rng_seed(o_rng* r, uint64_t seed) {
    uint64_t sm = seed;
    for (int k = 0; k < 4; ++k) {
        sm += 0x9e3779b97f4a7c15ull;
        uint64_t z = sm;
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        r->s[k] = z ^ (z >> 31);
    }
}

uint64_t o_rng_next(o_rng* r) {
    uint64_t* s = r->s;
    const uint64_t out = o_rotl(s[1] * 5u, 7) * 9u;
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = o_rotl(s[3], 45);
    return out;
}

/* Raw generator access for the known-answer tests: n outputs from a seed (splitmix
 * initialisation) or from an explicit state. */
void o_xoshiro_outputs(uint64_t seed, int n, uint64_t* out) {
    o_rng r;
    o_rng_seed(&r, seed);
    for (int i = 0; i < n; ++i) out[i] = o_rng_next(&r);
}
void o_xoshiro_outputs_state(const uint64_t* state, int n, uint64_t* out) {
    o_rng r;
    memcpy(r.s, state, sizeof r.s);
    for (int i = 0; i < n; ++i) out[i] = o_rng_next(&r);
}
void o_splitmix_state(uint64_t seed, uint64_t* state_out) {
    o_rng r;
    o_rng_seed(&r, seed);
    memcpy(state_out, r.s, sizeof r.s);
}

/* Box-Muller (turboquant.rs:388-394). */
static void o_box_muller(o_rng* r, float* z0, float* z1) {
    double u1 = (double)(o_rng_next(r) >> 11) / (double)(1ull << 53);
    if (u1 < 1e-15) u1 = 1e-15;
    const double u2 = (double)(o_rng_next(r) >> 11) / (double)(1ull << 53);
    const double rad = sqrt(-2.0 * log(u1));
    const double th = 2.0 * O_PI * u2;
    *z0 = (float)(rad * cos(th));
    *z1 = (float)(rad * sin(th));
}

/* The d x d Gaussian matrix the rotation is built from (turboquant.rs:308-320). */
void o_gaussian_matrix(int d, uint64_t seed, float* g) {
    o_rng r;
    o_rng_seed(&r, seed);
    const int64_t n = (int64_t)d * d;
    int64_t k = 0;
    while (k < n) {
        float z0, z1;
        o_box_muller(&r, &z0, &z1);
        g[k++] = z0;
        if (k < n) g[k++] = z1;
    }
}

/* generate_rotation_matrix (turboquant.rs:306-338): modified Gram-Schmidt on the columns
 * in f64 (qr_orthogonalize :399-438), row-major f32 out, then columns with a negative
 * diagonal entry negated. */
void o_rotation(int d, uint64_t seed, float* q) {
    const int64_t n = (int64_t)d * d;
    float* g = (float*)malloc(sizeof(float) * (size_t)n);
    double* cols = (double*)malloc(sizeof(double) * (size_t)n);
    o_gaussian_matrix(d, seed, g);
    for (int c = 0; c < d; ++c)
        for (int r = 0; r < d; ++r) cols[(int64_t)c * d + r] = (double)g[(int64_t)r * d + c];
    for (int i = 0; i < d; ++i) {
        double* ci = cols + (int64_t)i * d;
        double ss = 0.0;
        for (int r = 0; r < d; ++r) ss += ci[r] * ci[r];
        const double nrm = sqrt(ss);
        if (nrm > 1e-12)
            for (int r = 0; r < d; ++r) ci[r] /= nrm;
        for (int j = i + 1; j < d; ++j) {
            double* cj = cols + (int64_t)j * d;
            double dot = 0.0;
            for (int r = 0; r < d; ++r) dot += ci[r] * cj[r];
            for (int r = 0; r < d; ++r) cj[r] -= dot * ci[r];
        }
    }
    for (int r = 0; r < d; ++r)
        for (int c = 0; c < d; ++c) q[(int64_t)r * d + c] = (float)cols[(int64_t)c * d + r];
    for (int c = 0; c < d; ++c)
        if (q[(int64_t)c * d + c] < 0.0f)
            for (int r = 0; r < d; ++r) q[(int64_t)r * d + c] = -q[(int64_t)r * d + c];
    free(g);
    free(cols);
}

/* Nearest centroid, first minimum on a strict `<` (turboquant_compress.cu:121-130). */
int o_tq_code(float y, const float* c, int L) {
    float best = fabsf(y - c[0]);
    int idx = 0;
    for (int i = 1; i < L; ++i) {
        const float dd = fabsf(y - c[i]);
        if (dd < best) {
            best = dd;
            idx = i;
        }
    }
    return idx;
}

void o_tq_codes(const float* y, int64_t n, const float* c, int L, uint8_t* codes) {
    for (int64_t i = 0; i < n; ++i) codes[i] = (uint8_t)o_tq_code(y[i], c, L);
}

/* Bit packing of one head row of codes.
 * bits 2, 4, 8: the three layouts written out in turboquant_compress.cu:113-186.
 * other bits:   MSB-first bitstream, code d at stream bits [b*d, b*d + b), stream bit k
 *               being bit 7 - k%8 of byte k/8 (the generalisation of those layouts). */
void o_tq_pack_row(const uint8_t* codes, int hd, int bits, uint8_t* out) {
    const int pd = (hd * bits + 7) / 8;
    if (bits == 4) {
        for (int p = 0; p < (hd + 1) / 2; ++p) {
            const int i0 = codes[2 * p];
            const int i1 = 2 * p + 1 < hd ? codes[2 * p + 1] : 0;
            out[p] = (uint8_t)((i0 << 4) | (i1 & 0x0f));
        }
    } else if (bits == 2) {
        for (int q = 0; q < (hd + 3) / 4; ++q) {
            uint8_t v = 0;
            for (int s = 0; s < 4; ++s) {
                const int d = 4 * q + s;
                const int i = d < hd ? codes[d] : 0;
                v |= (uint8_t)(i << (6 - 2 * s));
            }
            out[q] = v;
        }
    } else if (bits == 8) {
        for (int d = 0; d < hd; ++d) out[d] = codes[d];
    } else {
        memset(out, 0, (size_t)pd);
        for (int d = 0; d < hd; ++d)
            for (int k = 0; k < bits; ++k) {
                const int bit = (codes[d] >> (bits - 1 - k)) & 1;
                const int sb = d * bits + k;
                out[sb / 8] |= (uint8_t)(bit << (7 - sb % 8));
            }
    }
}

/* The MSB-first bitstream for any bits (used to pin the generalisation at 2/4/8). */
void o_tq_pack_row_bitstream(const uint8_t* codes, int hd, int bits, uint8_t* out) {
    const int pd = (hd * bits + 7) / 8;
    memset(out, 0, (size_t)pd);
    for (int d = 0; d < hd; ++d)
        for (int k = 0; k < bits; ++k) {
            const int bit = (codes[d] >> (bits - 1 - k)) & 1;
            const int sb = d * bits + k;
            out[sb / 8] |= (uint8_t)(bit << (7 - sb % 8));
        }
}

/* Unpacking (turboquant_decompress.cu:40-73; attention_paged_tq.cu:39-54). */
int o_tq_unpack(const uint8_t* row, int d, int bits) {
    if (bits == 4) return d % 2 == 0 ? (row[d / 2] >> 4) & 0x0f : row[d / 2] & 0x0f;
    if (bits == 2) return (row[d / 4] >> (6 - (d % 4) * 2)) & 0x03;
    if (bits == 8) return row[d];
    int v = 0;
    for (int k = 0; k < bits; ++k) {
        const int sb = d * bits + k;
        v = (v << 1) | ((row[sb / 8] >> (7 - sb % 8)) & 1);
    }
    return v;
}

void o_tq_quantize_pack(const float* y, int64_t rows, int hd, const float* c, int L, int bits,
                        uint8_t* packed) {
    const int pd = (hd * bits + 7) / 8;
    uint8_t* codes = (uint8_t*)malloc((size_t)hd);
    for (int64_t r = 0; r < rows; ++r) {
        for (int d = 0; d < hd; ++d) codes[d] = (uint8_t)o_tq_code(y[r * hd + d], c, L);
        o_tq_pack_row(codes, hd, bits, packed + r * pd);
    }
    free(codes);
}

/* Rotated unit vectors and norms of turboquant_compress.cu:48-107, with the norm summed
 * sequentially as the CPU form of the same computation (turboquant.rs:1242-1251):
 * n = sqrt(sum x^2); x_hat = x * (1 / (n + 1e-8)); y_i = sum_j Pi[i][j] x_hat_j. */
void o_tq_rotate(const uint16_t* x16, int64_t rows, int hd, const float* rot, float* y,
                 uint16_t* norms16) {
    float* xh = (float*)malloc(sizeof(float) * (size_t)hd);
    for (int64_t r = 0; r < rows; ++r) {
        float ss = 0.0f;
        for (int j = 0; j < hd; ++j) {
            const float v = o_f16_to_f32(x16[r * hd + j]);
            ss += v * v;
        }
        const float nrm = sqrtf(ss);
        norms16[r] = o_f32_to_f16(nrm);
        const float inv = 1.0f / (nrm + 1e-8f);
        for (int j = 0; j < hd; ++j) xh[j] = o_f16_to_f32(x16[r * hd + j]) * inv;
        for (int i = 0; i < hd; ++i) {
            float dot = 0.0f;
            for (int j = 0; j < hd; ++j) dot += rot[(int64_t)i * hd + j] * xh[j];
            y[r * hd + i] = dot;
        }
    }
    free(xh);
}

/* Full compress: rotate, quantize, pack (turboquant_compress.cu:27-187). */
void o_tq_compress(const uint16_t* x16, int64_t rows, int hd, const float* rot, const float* c,
                   int L, int bits, uint8_t* packed, uint16_t* norms16, float* y_out) {
    float* y = y_out ? y_out : (float*)malloc(sizeof(float) * (size_t)(rows * hd));
    o_tq_rotate(x16, rows, hd, rot, y, norms16);
    o_tq_quantize_pack(y, rows, hd, c, L, bits, packed);
    if (!y_out) free(y);
}

/* Dequantize (turboquant_decompress.cu:40-94): y_hat = c[idx]; x_hat_i = sum_j Pi[j][i]
 * y_hat_j; out = f16(x_hat * f32(norm)). */
void o_tq_dequant(const uint8_t* packed, const uint16_t* norms16, int64_t rows, int hd,
                  const float* rot, const float* c, int bits, uint16_t* out16) {
    const int pd = (hd * bits + 7) / 8;
    float* yh = (float*)malloc(sizeof(float) * (size_t)hd);
    for (int64_t r = 0; r < rows; ++r) {
        for (int d = 0; d < hd; ++d) yh[d] = c[o_tq_unpack(packed + r * pd, d, bits)];
        const float nrm = o_f16_to_f32(norms16[r]);
        for (int i = 0; i < hd; ++i) {
            float dot = 0.0f;
            for (int j = 0; j < hd; ++j) dot += rot[(int64_t)j * hd + i] * yh[j];
            out16[r * hd + i] = o_f32_to_f16(dot * nrm);
        }
    }
    free(yh);
}

/* TurboQuant paged attention for one query token (attention_paged_tq.cu:79-257), query heads
 * [h_begin, h_end) only (out16 rows of the other heads are left untouched).
 * Pages live in pools: K packed page p at kp + p*skp bytes, layout [16][kvh][pdk]; norms at
 * kn + p*skn bytes, [16][kvh] fp16; likewise V. q16/out16: [qh][hd] fp16 for this token;
 * causal_len positions are attended through block_table.
 * The V accumulation visits positions in the outer loop: each coordinate's sum still adds
 * the positions in increasing order (attention_paged_tq.cu:222-243 sums over t per d), so
 * the result is the same as with the coordinate loop outside, with one pass over the rows. */
void o_tq_attention_heads(const uint16_t* q16, const int32_t* block_table, int causal_len,
                          const uint8_t* kp, const uint8_t* kn, const uint8_t* vp,
                          const uint8_t* vn, int64_t skp, int64_t skn, int64_t svp, int64_t svn,
                          const float* krot, const float* vrot, const float* kc, const float* vc,
                          int kbits, int vbits, int qh, int kvh, int hd, int h_begin, int h_end,
                          uint16_t* out16) {
    const int G = qh / kvh;
    const int pdk = (hd * kbits + 7) / 8, pdv = (hd * vbits + 7) / 8;
    const float scale = 1.0f / sqrtf((float)hd);
    float* qrot = (float*)malloc(sizeof(float) * (size_t)hd);
    float* acc = (float*)malloc(sizeof(float) * (size_t)hd);
    float* sc = (float*)malloc(sizeof(float) * (size_t)(causal_len > 0 ? causal_len : 1));
    if (h_begin < 0) h_begin = 0;
    if (h_end > qh) h_end = qh;
    for (int h = h_begin; h < h_end; ++h) {
        const int kvhd = h / G;
        for (int i = 0; i < hd; ++i) {
            float dot = 0.0f;
            for (int j = 0; j < hd; ++j)
                dot += krot[(int64_t)i * hd + j] * o_f16_to_f32(q16[(int64_t)h * hd + j]);
            qrot[i] = dot;
        }
        float mx = -3.402823466e38f;
        for (int t = 0; t < causal_len; ++t) {
            const int page = block_table[t / 16], off = t % 16;
            const uint8_t* row = kp + (int64_t)page * skp + ((int64_t)off * kvh + kvhd) * pdk;
            const float kn_ = o_f16_to_f32(((const uint16_t*)(kn + (int64_t)page * skn))[off * kvh + kvhd]);
            float dot = 0.0f;
            for (int d = 0; d < hd; ++d) dot += qrot[d] * kc[o_tq_unpack(row, d, kbits)];
            dot *= kn_ * scale;
            sc[t] = dot;
            if (dot > mx) mx = dot;
        }
        float sum = 0.0f;
        for (int t = 0; t < causal_len; ++t) {
            sc[t] = expf(sc[t] - mx);
            sum += sc[t];
        }
        const float inv = 1.0f / sum;
        for (int t = 0; t < causal_len; ++t) sc[t] *= inv;
        for (int d = 0; d < hd; ++d) acc[d] = 0.0f;
        for (int t = 0; t < causal_len; ++t) {
            const int page = block_table[t / 16], off = t % 16;
            const uint8_t* row = vp + (int64_t)page * svp + ((int64_t)off * kvh + kvhd) * pdv;
            const float vn_ = o_f16_to_f32(((const uint16_t*)(vn + (int64_t)page * svn))[off * kvh + kvhd]);
            for (int d = 0; d < hd; ++d) acc[d] += sc[t] * vc[o_tq_unpack(row, d, vbits)] * vn_;
        }
        for (int i = 0; i < hd; ++i) {
            float dot = 0.0f;
            for (int j = 0; j < hd; ++j) dot += vrot[(int64_t)j * hd + i] * acc[j];
            out16[(int64_t)h * hd + i] = o_f32_to_f16(dot);
        }
    }
    free(qrot);
    free(acc);
    free(sc);
}

/* Every query head of one token. */
void o_tq_attention(const uint16_t* q16, const int32_t* block_table, int causal_len,
                    const uint8_t* kp, const uint8_t* kn, const uint8_t* vp, const uint8_t* vn,
                    int64_t skp, int64_t skn, int64_t svp, int64_t svn, const float* krot,
                    const float* vrot, const float* kc, const float* vc, int kbits, int vbits,
                    int qh, int kvh, int hd, uint16_t* out16) {
    o_tq_attention_heads(q16, block_table, causal_len, kp, kn, vp, vn, skp, skn, svp, svn, krot,
                         vrot, kc, vc, kbits, vbits, qh, kvh, hd, 0, qh, out16);
}

/* FP16 paged GQA attention for one query token (attention_paged.cu:36-170).
 * Pages live in pools: K page p at kpool + p*skp bytes, layout [16][kvh][hd] fp16; likewise V.
 * q16/out16: [qh][hd] fp16 for this token; causal_len positions are attended through
 * block_table. Per head: score_t = (sum_d q_d k_d, in d order) * (1/sqrt(hd)) (:61-70; the
 * kernel's rsqrtf), max, e_t = exp(score_t - max), sum, p_t = e_t / sum (:107-134), then
 * out_d = half(sum_t p_t v_td, in t order) (:138-150). causal_len 0 gives zeros. */
void o_paged_attention(const uint16_t* q16, const int32_t* block_table, int causal_len,
                       const uint8_t* kpool, const uint8_t* vpool, int64_t skp, int64_t svp,
                       int qh, int kvh, int hd, uint16_t* out16) {
    const int G = qh / kvh;
    const float scale = 1.0f / sqrtf((float)hd);
    float* sc = (float*)malloc(sizeof(float) * (size_t)(causal_len > 0 ? causal_len : 1));
    for (int h = 0; h < qh; ++h) {
        const int kvhd = h / G;
        const uint16_t* qv = q16 + (int64_t)h * hd;
        float mx = -3.402823466e38f;
        for (int t = 0; t < causal_len; ++t) {
            const int page = block_table[t / 16], off = t % 16;
            const uint16_t* k = (const uint16_t*)(kpool + (int64_t)page * skp) +
                                ((int64_t)off * kvh + kvhd) * hd;
            float dot = 0.0f;
            for (int d = 0; d < hd; ++d) dot += o_f16_to_f32(qv[d]) * o_f16_to_f32(k[d]);
            dot *= scale;
            sc[t] = dot;
            if (dot > mx) mx = dot;
        }
        float sum = 0.0f;
        for (int t = 0; t < causal_len; ++t) {
            sc[t] = expf(sc[t] - mx);
            sum += sc[t];
        }
        const float inv = 1.0f / sum;
        for (int t = 0; t < causal_len; ++t) sc[t] *= inv;
        for (int d = 0; d < hd; ++d) {
            float a = 0.0f;
            for (int t = 0; t < causal_len; ++t) {
                const int page = block_table[t / 16], off = t % 16;
                const uint16_t* v = (const uint16_t*)(vpool + (int64_t)page * svp) +
                                    ((int64_t)off * kvh + kvhd) * hd;
                a += sc[t] * o_f16_to_f32(v[d]);
            }
            out16[(int64_t)h * hd + d] = o_f32_to_f16(a);
        }
    }
    free(sc);
}
