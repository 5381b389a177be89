// Exhaustive host check of poorgrad_amd/csrc/faithful_math.h against the host
// C library: every one of the 2^32 single-precision inputs (or a range of
// them), split over threads. Also recomputes the tables from their
// definitions, and hashes the host libm's outputs for comparison with the
// device build of the same functions.
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <string.h>

#include <vector>

#include "../../poorgrad_amd/csrc/faithful_math.h"

namespace {

using namespace topos_faithful;

float host_libm(int function, float x) {
  switch (function) {
    case 0: return expf(x);
    case 1: return logf(x);
    case 2: return tanhf(x);
    default: return sqrtf(x);
  }
}

float restated(int function, float x) {
  switch (function) {
    case 0: return exp_f32(x);
    case 1: return ln_f32(x);
    case 2: return tanh_f32(x);
    default: return __builtin_sqrtf(x);
  }
}

// NaN results compare as a class: payloads are not part of the contract.
uint32_t canonical(float y) { return y != y ? 0x7fc00000u : bits_of(y); }

// Order-independent digest term of one (input, output) pair.
uint64_t digest(uint32_t input, uint32_t output) {
  uint64_t z = ((uint64_t)input << 32) | output;
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

struct Work {
  int function;
  uint64_t begin, end;
  int64_t mismatches;
  uint32_t first_bad;
  uint64_t hash;
  int mode;  // 0: compare, 1: hash the host libm, 2: write the host libm's bits
  uint32_t *out;
  uint64_t out_base;
};

void *run(void *arg) {
  Work *w = static_cast<Work *>(arg);
  for (uint64_t u = w->begin; u < w->end; ++u) {
    const float x = float_of((uint32_t)u);
    const uint32_t host = canonical(host_libm(w->function, x));
    if (w->mode == 2) {
      w->out[u - w->out_base] = host;
    } else if (w->mode == 1) {
      w->hash += digest((uint32_t)u, host);
    } else if (host != canonical(restated(w->function, x))) {
      if (w->mismatches == 0) w->first_bad = (uint32_t)u;
      ++w->mismatches;
    }
  }
  return nullptr;
}

std::vector<Work> spread(int function, uint64_t begin, uint64_t end, int threads, int mode,
                         uint32_t *out = nullptr) {
  if (threads < 1) threads = 1;
  std::vector<Work> work(threads);
  std::vector<pthread_t> ids(threads);
  const uint64_t span = (end - begin + threads - 1) / threads;
  for (int t = 0; t < threads; ++t) {
    const uint64_t b = begin + span * t;
    const uint64_t e = b + span < end ? b + span : end;
    work[t] = Work{function, b < end ? b : end, e, 0, 0, 0, mode, out, begin};
    pthread_create(&ids[t], nullptr, run, &work[t]);
  }
  for (int t = 0; t < threads; ++t) pthread_join(ids[t], nullptr);
  return work;
}

}  // namespace

extern "C" {

// Counts inputs in [begin, end) where the restated function differs from the
// host libm; the first differing input's bits go to *first_bad.
int64_t faithful_check(int function, uint64_t begin, uint64_t end, int threads, uint32_t *first_bad) {
  int64_t total = 0;
  bool seen = false;
  for (const Work &w : spread(function, begin, end, threads, 0)) {
    if (w.mismatches && !seen) {
      *first_bad = w.first_bad;
      seen = true;
    }
    total += w.mismatches;
  }
  return total;
}

// Wrapping sum of digest(input, host libm output) over [begin, end).
uint64_t host_libm_digest(int function, uint64_t begin, uint64_t end, int threads) {
  uint64_t hash = 0;
  for (const Work &w : spread(function, begin, end, threads, 1)) hash += w.hash;
  return hash;
}

// Writes the host libm's result bits (NaN canonicalised) for the inputs
// whose bit patterns are begin..begin+count-1 into out[0..count).
void host_libm_range(int function, uint64_t begin, uint64_t count, uint32_t *out, int threads) {
  spread(function, begin, begin + count, threads, 2, out);
}

// splitmix64, for reproducible input streams.
static uint64_t mix(uint64_t *state) {
  uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// The (x, y) pair number `index` of input family `family` for powf:
//   0: both operands uniform over all 2^32 bit patterns (specials, subnormals);
//   1: x = 2^u with u uniform in [-150, 128), y uniform in [-40, 40];
//   2: x negative with an integer or half-integer y in [-64, 64];
//   3: x within 2^-10 of 1, |y| up to 2^20;
//   4: y log2 x near the overflow and underflow edges (126, 128, -126, -149, -150);
//   5: y an integer or a small dyadic in [-8, 8], x uniform in [2^-4, 2^4].
void pow_pair(int family, uint64_t seed, uint64_t index, float *x, float *y) {
  uint64_t state = seed * 0x100000001B3ull + index * 0x9E3779B97F4A7C15ull + (uint64_t)family;
  const uint64_t a = mix(&state), b = mix(&state);
  const double ua = (double)(a >> 11) / 9007199254740992.0, ub = (double)(b >> 11) / 9007199254740992.0;
  switch (family) {
    case 0:
      *x = float_of((uint32_t)a);
      *y = float_of((uint32_t)b);
      return;
    case 1:
      *x = (float)exp2(-150.0 + 278.0 * ua);
      *y = (float)(-40.0 + 80.0 * ub);
      return;
    case 2: {
      *x = -(float)exp2(-20.0 + 40.0 * ua);
      const int64_t n = (int64_t)(b % 257) - 128;
      *y = (float)n * ((b >> 32) & 1 ? 0.5f : 1.0f);
      return;
    }
    case 3:
      *x = (float)(1.0 + (ua - 0.5) * 0x1p-9);
      *y = (float)((ub - 0.5) * 0x1p21);
      return;
    case 4: {
      static const double edges[5] = {126.0, 128.0, -126.0, -149.0, -150.0};
      const double edge = edges[b % 5] + ((double)((b >> 8) % 2001) - 1000.0) * 1e-7;
      float xf = (float)exp2(-8.0 + 16.0 * ua);
      if (xf == 1.0f) xf = 2.0f;
      *x = xf;
      *y = (float)(edge / log2((double)xf));
      return;
    }
    default:
      *x = (float)exp2(-4.0 + 8.0 * ua);
      *y = (float)((int64_t)(b % 1025) - 512) / 64.0f;
      return;
  }
}

struct PowWork {
  int family;
  uint64_t seed, begin, end;
  int64_t mismatches;
  float bad_x, bad_y;
};

void *run_pow(void *arg) {
  PowWork *w = static_cast<PowWork *>(arg);
  for (uint64_t i = w->begin; i < w->end; ++i) {
    float x, y;
    pow_pair(w->family, w->seed, i, &x, &y);
    if (canonical(powf(x, y)) != canonical(pow_f32(x, y))) {
      if (w->mismatches == 0) {
        w->bad_x = x;
        w->bad_y = y;
      }
      ++w->mismatches;
    }
  }
  return nullptr;
}

// Counts pairs 0..count-1 of a family where the restated powf differs from
// the host libm's (NaN as a class); the first differing pair goes to bad[0..2).
int64_t pow_check(int family, uint64_t seed, uint64_t count, int threads, float *bad) {
  if (threads < 1) threads = 1;
  std::vector<PowWork> work(threads);
  std::vector<pthread_t> ids(threads);
  const uint64_t span = (count + threads - 1) / threads;
  for (int t = 0; t < threads; ++t) {
    const uint64_t b = span * t < count ? span * t : count;
    const uint64_t e = b + span < count ? b + span : count;
    work[t] = PowWork{family, seed, b, e, 0, 0.0f, 0.0f};
    pthread_create(&ids[t], nullptr, run_pow, &work[t]);
  }
  int64_t total = 0;
  bool seen = false;
  for (int t = 0; t < threads; ++t) {
    pthread_join(ids[t], nullptr);
    if (work[t].mismatches && !seen) {
      bad[0] = work[t].bad_x;
      bad[1] = work[t].bad_y;
      seen = true;
    }
    total += work[t].mismatches;
  }
  return total;
}

// Writes pairs 0..count-1 of a family and the host libm's powf of each (NaN
// canonicalised), for comparison with the device build.
void pow_pairs(int family, uint64_t seed, uint64_t count, float *x, float *y, uint32_t *host) {
  for (uint64_t i = 0; i < count; ++i) {
    pow_pair(family, seed, i, &x[i], &y[i]);
    host[i] = canonical(powf(x[i], y[i]));
  }
}

// Recomputes the exp table (bits(RN(2^(i/32))) - (i << 52)/32) and the log
// table's logc = RN(-log(invc)) in extended precision; returns the number of
// entries that disagree with faithful_math.h.
int faithful_tables_check(void) {
  int bad = 0;
  for (int i = 0; i < 32; ++i) {
    const double v = (double)exp2l((long double)i / 32.0L);
    const uint64_t expected = bits_of(v) - (((uint64_t)i << 52) / 32);
    if (expected != kExpTableHost[i]) ++bad;
  }
  for (int i = 0; i < 16; ++i) {
    const double logc = (double)logl(1.0L / (long double)kLogTableHost[i].invc);
    if (logc != kLogTableHost[i].logc) ++bad;
    // powf's log2 table: the same 1/c, and RN(log2 c).
    if (kLog2TableHost[i].invc != kLogTableHost[i].invc) ++bad;
    const double log2c = (double)log2l(1.0L / (long double)kLog2TableHost[i].invc);
    if (log2c != kLog2TableHost[i].logc) ++bad;
  }
  return bad;
}

}  // extern "C"
