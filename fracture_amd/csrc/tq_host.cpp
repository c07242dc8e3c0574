// Host-side TurboQuant tables and the RoPE frequency table, computed on the CPU exactly as
// the reference does before uploading them (crates/fracture-core/src/turboquant.rs:99-438,
// backends/fracture-cuda/src/lib.rs:133-139). The operations and their order follow the
// Rust source so that, with IEEE double arithmetic, glibc's exp/log/sin/cos and no FMA
// contraction (this file is built with -ffp-contract=off), the tables are bit-identical.
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <vector>

#include "fracture_hip.h"

namespace {

const double kPi = 3.14159265358979323846;

// turboquant.rs:166-168
double gaussian_pdf(double x, double sigma2) {
    return (1.0 / sqrt(2.0 * kPi * sigma2)) * exp(-x * x / (2.0 * sigma2));
}

// turboquant.rs:171-180, composite Simpson with an even number of intervals.
template <class F>
double integrate_simpson(F f, double a, double b, int n) {
    if (n % 2 == 1) n += 1;
    const double h = (b - a) / (double)n;
    double sum = f(a) + f(b);
    for (int i = 1; i < n; ++i) {
        const double x = a + (double)i * h;
        sum += (i % 2 == 0) ? 2.0 * f(x) : 4.0 * f(x);
    }
    return sum * h / 3.0;
}

// SplitMix64-seeded Xoshiro256** (turboquant.rs:349-385).
struct Xoshiro256 {
    uint64_t s[4];
    explicit Xoshiro256(uint64_t seed) {
        uint64_t sm = seed;
        for (int k = 0; k < 4; ++k) {
            sm += 0x9e3779b97f4a7c15ull;
            uint64_t z = sm;
            z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
            z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
            z ^= z >> 31;
            s[k] = z;
        }
    }
    static uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
    uint64_t next_u64() {
        const uint64_t result = rotl(s[1] * 5, 7) * 9;
        const uint64_t t = s[1] << 17;
        s[2] ^= s[0];
        s[3] ^= s[1];
        s[1] ^= s[2];
        s[0] ^= s[3];
        s[2] ^= t;
        s[3] = rotl(s[3], 45);
        return result;
    }
    double next_f64() { return (double)(next_u64() >> 11) / (double)(1ull << 53); }
};

// turboquant.rs:388-394
void box_muller(Xoshiro256& rng, float* z0, float* z1) {
    double u1 = rng.next_f64();
    u1 = fmax(u1, 1e-15);
    const double u2 = rng.next_f64();
    const double r = sqrt(-2.0 * log(u1));
    const double theta = 2.0 * kPi * u2;
    *z0 = (float)(r * cos(theta));
    *z1 = (float)(r * sin(theta));
}

}  // namespace

extern "C" {

size_t fhip_tq_packed_dim_per_head(size_t head_dim, int bits) {
    return (head_dim * (size_t)bits + 7) / 8;
}

// LloydMaxCodebook::compute (turboquant.rs:186-250).
int fhip_tq_codebook(int dim, int bits, float* centroids_out, float* boundaries_out) {
    if (dim <= 0 || bits < 1 || bits > 8 || !centroids_out) return FHIP_ERR_INVALID_SHAPE;
    const int n_levels = 1 << bits;
    const double sigma2 = 1.0 / (double)dim;
    const double sigma = sqrt(sigma2);
    const double lo = -3.5 * sigma;
    const double hi = 3.5 * sigma;
    std::vector<double> c(n_levels), nc(n_levels), bnd(n_levels - 1);
    for (int i = 0; i < n_levels; ++i)
        c[i] = lo + (hi - lo) * ((double)i + 0.5) / (double)n_levels;
    const int max_iter = 200;
    const double tol = 1e-10;
    const int n_quad = 500;
    for (int it = 0; it < max_iter; ++it) {
        for (int i = 0; i < n_levels - 1; ++i) bnd[i] = (c[i] + c[i + 1]) / 2.0;
        const double edges_lo = lo * 3.0;
        const double edges_hi = hi * 3.0;
        double max_shift = 0.0;
        for (int i = 0; i < n_levels; ++i) {
            const double a = i == 0 ? edges_lo : bnd[i - 1];
            const double b = i == n_levels - 1 ? edges_hi : bnd[i];
            const double num = integrate_simpson(
                [sigma2](double x) { return x * gaussian_pdf(x, sigma2); }, a, b, n_quad);
            const double den =
                integrate_simpson([sigma2](double x) { return gaussian_pdf(x, sigma2); }, a, b,
                                  n_quad);
            const double new_c = fabs(den) > 1e-15 ? num / den : c[i];
            max_shift = fmax(max_shift, fabs(new_c - c[i]));
            nc[i] = new_c;
        }
        c.swap(nc);
        if (max_shift < tol) break;
    }
    for (int i = 0; i < n_levels; ++i) centroids_out[i] = (float)c[i];
    if (boundaries_out)
        for (int i = 0; i < n_levels - 1; ++i) boundaries_out[i] = (float)((c[i] + c[i + 1]) / 2.0);
    return FHIP_OK;
}

// generate_rotation_matrix (turboquant.rs:306-338) with qr_orthogonalize (:399-438).
int fhip_tq_rotation_matrix(int d, uint64_t seed, float* out) {
    if (d <= 0 || !out) return FHIP_ERR_INVALID_SHAPE;
    Xoshiro256 rng(seed);
    const size_t n = (size_t)d * d;
    std::vector<float> g;
    g.reserve(n + 1);
    const size_t pairs = (n + 1) / 2;
    for (size_t p = 0; p < pairs; ++p) {
        float z0, z1;
        box_muller(rng, &z0, &z1);
        g.push_back(z0);
        if (g.size() < n) g.push_back(z1);
    }
    // Modified Gram-Schmidt on the columns, in f64.
    std::vector<double> cols(n);  // cols[col * d + row]
    for (int col = 0; col < d; ++col)
        for (int row = 0; row < d; ++row) cols[(size_t)col * d + row] = (double)g[(size_t)row * d + col];
    for (int i = 0; i < d; ++i) {
        double* ci = &cols[(size_t)i * d];
        double ss = 0.0;
        for (int r = 0; r < d; ++r) ss += ci[r] * ci[r];
        const double norm = sqrt(ss);
        if (norm > 1e-12)
            for (int r = 0; r < d; ++r) ci[r] /= norm;
        for (int j = i + 1; j < d; ++j) {
            double* cj = &cols[(size_t)j * d];
            double dot = 0.0;
            for (int r = 0; r < d; ++r) dot += ci[r] * cj[r];
            for (int r = 0; r < d; ++r) cj[r] -= dot * ci[r];
        }
    }
    for (int row = 0; row < d; ++row)
        for (int col = 0; col < d; ++col)
            out[(size_t)row * d + col] = (float)cols[(size_t)col * d + row];
    // Flip columns whose diagonal element is negative.
    for (int col = 0; col < d; ++col) {
        if (out[(size_t)col * d + col] < 0.0f)
            for (int row = 0; row < d; ++row) out[(size_t)row * d + col] = -out[(size_t)row * d + col];
    }
    return FHIP_OK;
}

// rotation_seeds (turboquant.rs:341-345).
void fhip_tq_rotation_seeds(uint64_t base_seed, uint64_t layer, uint64_t* k_seed,
                            uint64_t* v_seed) {
    if (k_seed) *k_seed = base_seed + layer * 1000ull;
    if (v_seed) *v_seed = base_seed + layer * 1000ull + 500ull;
}

// precompute_rope_freqs table (lib.rs:134-139): freq[i] = 1 / (theta^(2i/hd) as f32).
void fhip_rope_freqs(int head_dim, double theta, float* out) {
    const int half = head_dim / 2;
    for (int i = 0; i < half; ++i)
        out[i] = 1.0f / (float)pow(theta, 2.0 * (double)i / (double)head_dim);
}

const char* fhip_version(void) { return "fracture-hip 0.1.0 (gfx950)"; }

}  // extern "C"
