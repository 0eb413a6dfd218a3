// synthetic.hip -- deterministic synthetic checkpoint values (host code).
//
// The benchmark configurations use random-init BF16 weights ~N(0, stddev)
// because the real YuE2 checkpoint is downloaded by the reference
// (src/checkpoint.rs:16-161) and is not available offline.  Values come from
// a counter-based generator so they can be produced in parallel and are the
// same on every machine:
//   key   = SplitMix64(SplitMix64(seed) + tensor)
//   bits  = SplitMix64(key + pair)                       (Steele, Lea, Flood 2014)
//   u1    = (bits[63:40] + 1) / 2^24 in (0, 1],  u2 = bits[39:16] / 2^24
//   z0,z1 = sqrt(-2 ln u1) * (cos, sin)(2 pi u2)         (Box-Muller 1958)
//   w     = rb((float)(stddev * z))
// ln, sin and cos are evaluated here from their series with IEEE operations
// only, so no platform libm enters the values.
#include <algorithm>
#include <thread>
#include <vector>

#include "../../include/yue2_hip.h"
#include "y2_math.h"

namespace {

uint64_t splitmix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

double ln_positive(double u) {
    int k;
    const double m = y2::split_log_arg(u, &k);
    const double kd = (double)k;
    return __builtin_fma(kd, 0x1.62e42fefa3800p-1, y2::log_core(m) + kd * 0x1.ef35793c76730p-45);
}

// sin/cos of t in [0, pi/4] from their Taylor series (truncation < 1e-19).
void sincos_small(double t, double* s, double* c) {
    const double z = t * t;
    double ps = -1.0 / 121645100408832000.0;  // -1/19!
    ps = __builtin_fma(ps, z, 1.0 / 355687428096000.0);
    ps = __builtin_fma(ps, z, -1.0 / 1307674368000.0);
    ps = __builtin_fma(ps, z, 1.0 / 6227020800.0);
    ps = __builtin_fma(ps, z, -1.0 / 39916800.0);
    ps = __builtin_fma(ps, z, 1.0 / 362880.0);
    ps = __builtin_fma(ps, z, -1.0 / 5040.0);
    ps = __builtin_fma(ps, z, 1.0 / 120.0);
    ps = __builtin_fma(ps, z, -1.0 / 6.0);
    *s = __builtin_fma(t * z, ps, t);
    double pc = 1.0 / 6402373705728000.0;  // 1/18!
    pc = __builtin_fma(pc, z, -1.0 / 20922789888000.0);
    pc = __builtin_fma(pc, z, 1.0 / 87178291200.0);
    pc = __builtin_fma(pc, z, -1.0 / 479001600.0);
    pc = __builtin_fma(pc, z, 1.0 / 3628800.0);
    pc = __builtin_fma(pc, z, -1.0 / 40320.0);
    pc = __builtin_fma(pc, z, 1.0 / 720.0);
    pc = __builtin_fma(pc, z, -1.0 / 24.0);
    pc = __builtin_fma(pc, z, 0.5);
    *c = __builtin_fma(-z, pc, 1.0);
}

// (sin, cos)(2 pi u) for u in [0, 1): quadrant from 4u (exact), then the
// reflected argument in [0, pi/4].
void sincos_2pi(double u, double* s, double* c) {
    const double v = 4.0 * u;
    const double q = __builtin_floor(v);
    const double f = v - q;
    const int quadrant = (int)q & 3;
    constexpr double half_pi = 0x1.921fb54442d18p+0;
    double sf, cf;
    if (f <= 0.5) {
        sincos_small(f * half_pi, &sf, &cf);
    } else {
        double sg, cg;
        sincos_small((1.0 - f) * half_pi, &sg, &cg);
        sf = cg;
        cf = sg;
    }
    switch (quadrant) {
        case 0: *s = sf; *c = cf; break;
        case 1: *s = cf; *c = -sf; break;
        case 2: *s = -sf; *c = -cf; break;
        default: *s = -cf; *c = sf; break;
    }
}

void fill_range(uint16_t* out, size_t n, uint64_t key, double stddev, size_t pair_begin,
                size_t pair_end) {
    for (size_t j = pair_begin; j < pair_end; ++j) {
        const uint64_t bits = splitmix64(key + j);
        const double u1 = (double)((bits >> 40) + 1) * 0x1.0p-24;
        const double u2 = (double)((bits >> 16) & 0xffffffull) * 0x1.0p-24;
        const double r = __builtin_sqrt(-2.0 * ln_positive(u1));
        double s, c;
        sincos_2pi(u2, &s, &c);
        const size_t i = 2 * j;
        out[i] = y2::bf16_bits(y2::rb((float)(stddev * (r * c))));
        if (i + 1 < n) out[i + 1] = y2::bf16_bits(y2::rb((float)(stddev * (r * s))));
    }
}

}  // namespace

extern "C" void yue2_hip_synthetic_bf16(uint16_t* out, size_t n, uint64_t seed, uint64_t tensor,
                                        float stddev, int32_t threads) {
    if (!out || n == 0) return;
    const uint64_t key = splitmix64(splitmix64(seed) + tensor);
    const size_t pairs = (n + 1) / 2;
    int t = threads > 0 ? threads : (int)std::max(1u, std::thread::hardware_concurrency());
    t = (int)std::min<size_t>((size_t)std::min(t, 64), std::max<size_t>(1, pairs / 65536));
    if (t <= 1) {
        fill_range(out, n, key, (double)stddev, 0, pairs);
        return;
    }
    std::vector<std::thread> pool;
    const size_t per = (pairs + t - 1) / t;
    for (int i = 0; i < t; ++i) {
        const size_t b = std::min(pairs, per * i), e = std::min(pairs, per * (i + 1));
        pool.emplace_back(fill_range, out, n, key, (double)stddev, b, e);
    }
    for (auto& th : pool) th.join();
}
