// Per-move root operations on the device (gfx950): the visit-count policy of every root,
// move selection with a temperature, and root Dirichlet noise.
//
// Reference:
//   policy        MCTS._extract_policy (python/mcts/core/mcts.py:1069-1137)
//   selection     MCTS.select_action (mcts.py:1167-1203): temperature 0 takes the first
//                 maximum (np.argmax); otherwise p^(1/T) is normalised and sampled
//                 (np.random.choice: cumulative sums, normalised by the last, first entry
//                 above the uniform draw)
//   root noise    optimized_wave_search.py:387-392 (np.random.dirichlet at root expansion);
//                 the GPU kernel of mcts_kernels.cu:649-754
//
// The random draws come from a counter-based stream instead of numpy's global generator. The
// stream is SplitMix64 keyed by (seed, counter, tree, item), so any call can be reproduced from
// its arguments and restated on the host.
//   - Gamma variates: Marsaglia and Tsang's method ("A simple method for generating gamma
//     variables", ACM TOMS 26(3), 2000). Shape alpha < 1 is boosted as G(alpha+1) * U^(1/alpha).
//   - Normal variates: Marsaglia's polar method.
//   - log and exp: evaluated here by textbook methods, so that the host restatement, which runs
//     the same operation sequence, gives the same bits. exp uses a Cody-Waite reduction by ln 2
//     and a degree-13 Taylor polynomial. log splits the exponent and uses the atanh series in
//     s = (m-1)/(m+1).
//   - Everything else is +, -, *, / and sqrt, which IEEE rounds correctly on both sides.
#include "omq_common.h"

namespace omq {

// ---- double-precision log and exp (identical operation sequence on the host side) ----------
constexpr double kLn2Hi = 0x1.62e42feep-1;        // ln 2 to 32 significant bits
constexpr double kLn2Lo = 0x1.a39ef35793c76p-33;  // ln 2 - kLn2Hi
constexpr double kInvLn2 = 1.0 / 0.6931471805599453;
constexpr double kSqrt2 = 0x1.6a09e667f3bcdp+0;

__device__ inline double pow2i(int k) {  // 2^k for -1022 <= k <= 1023
  return __longlong_as_double((long long)(k + 1023) << 52);
}

__device__ inline double exp_cw_d(double x) {
  if (x < -745.0) return 0.0;
  if (x > 709.0) return __longlong_as_double(0x7FF0000000000000LL);
  const double kf = floor(x * kInvLn2 + 0.5);
  const int k = (int)kf;
  const double r = (x - kf * kLn2Hi) - kf * kLn2Lo;
  double p = 1.0 / 6227020800.0;  // 1/13!
  p = p * r + 1.0 / 479001600.0;
  p = p * r + 1.0 / 39916800.0;
  p = p * r + 1.0 / 3628800.0;
  p = p * r + 1.0 / 362880.0;
  p = p * r + 1.0 / 40320.0;
  p = p * r + 1.0 / 5040.0;
  p = p * r + 1.0 / 720.0;
  p = p * r + 1.0 / 120.0;
  p = p * r + 1.0 / 24.0;
  p = p * r + 1.0 / 6.0;
  p = p * r + 0.5;
  p = p * r + 1.0;
  p = p * r + 1.0;
  if (k < -1021) return (p * pow2i(k + 1000)) * pow2i(-1000);
  return p * pow2i(k);
}

__device__ inline double log_cw_d(double x) {  // x > 0, finite
  long long b = __double_as_longlong(x);
  int e = 0;
  if ((b >> 52) == 0) {  // subnormal: scale into the normal range
    x = x * 0x1p54;
    b = __double_as_longlong(x);
    e = -54;
  }
  e += (int)((b >> 52) & 0x7FF) - 1023;
  double m = __longlong_as_double((b & 0x000FFFFFFFFFFFFFLL) | 0x3FF0000000000000LL);  // [1, 2)
  if (m > kSqrt2) {
    m = m * 0.5;
    e += 1;
  }
  const double s = (m - 1.0) / (m + 1.0);
  const double z = s * s;
  double p = 1.0 / 23.0;
  p = p * z + 1.0 / 21.0;
  p = p * z + 1.0 / 19.0;
  p = p * z + 1.0 / 17.0;
  p = p * z + 1.0 / 15.0;
  p = p * z + 1.0 / 13.0;
  p = p * z + 1.0 / 11.0;
  p = p * z + 1.0 / 9.0;
  p = p * z + 1.0 / 7.0;
  p = p * z + 1.0 / 5.0;
  p = p * z + 1.0 / 3.0;
  p = p * z + 1.0;
  const double ed = (double)e;
  return (ed * kLn2Lo + 2.0 * s * p) + ed * kLn2Hi;
}

// ---- counter-based stream -----------------------------------------------------------------
struct Stream {
  uint64_t base;
  uint64_t j;
};

__device__ inline Stream make_stream(uint64_t seed, uint64_t counter, int t, int item) {
  Stream s;
  s.base = splitmix64(splitmix64(splitmix64(seed) ^ counter) ^
                      (((uint64_t)(uint32_t)t << 32) | (uint32_t)item));
  s.j = 0;
  return s;
}

// uniform in (0, 1): (top 53 bits + 1/2) * 2^-53
__device__ inline double uniform_open(Stream& s) {
  const uint64_t b = splitmix64(s.base + s.j * kGolden);
  s.j += 1;
  return ((double)(b >> 11) + 0.5) * 0x1p-53;
}

__device__ inline double normal_polar(Stream& s) {
  for (;;) {
    const double u = 2.0 * uniform_open(s) - 1.0;
    const double v = 2.0 * uniform_open(s) - 1.0;
    const double q = u * u + v * v;
    if (q > 0.0 && q < 1.0) return u * sqrt(-2.0 * log_cw_d(q) / q);
  }
}

__device__ inline double gamma_mt(double alpha, Stream& s) {
  const bool boost = alpha < 1.0;
  const double a = boost ? alpha + 1.0 : alpha;
  const double d = a - 1.0 / 3.0;
  const double c = 1.0 / sqrt(9.0 * d);
  double x, v;
  for (;;) {
    do {
      x = normal_polar(s);
      v = 1.0 + c * x;
    } while (v <= 0.0);
    v = v * v * v;
    const double u = uniform_open(s);
    const double x2 = x * x;
    if (u < 1.0 - 0.0331 * (x2 * x2)) break;
    if (log_cw_d(u) < 0.5 * x2 + d * (1.0 - v + log_cw_d(v))) break;
  }
  double g = d * v;
  if (boost) g = g * exp_cw_d(log_cw_d(uniform_open(s)) / alpha);
  return g;
}

// ---- root policy ----------------------------------------------------------------------------
constexpr int kRootThreads = 256;

__global__ __launch_bounds__(kRootThreads) void root_policy_kernel(omq_forest f, double* pol) {
  __shared__ unsigned long long s_tot;
  const int t = blockIdx.x;
  const int tid = threadIdx.x;
  const int A = f.num_actions;
  const int64_t tb = (int64_t)t * f.capacity;
  double* row = pol + (int64_t)t * A;
  const int k = f.num_children[tb];
  const int first = f.first_child[tb];
  if (tid == 0) s_tot = 0ull;
  __syncthreads();
  unsigned long long part = 0;
  if (first >= 0)
    for (int j = tid; j < k; j += kRootThreads) part += (unsigned long long)f.visit_counts[tb + first + 1 + j];
  if (part) atomicAdd(&s_tot, part);
  __syncthreads();
  const unsigned long long tot = s_tot;
  const bool no_children = k <= 0 || first < 0;
  const double fill = no_children ? 1.0 / (double)A : 0.0;
  for (int a = tid; a < A; a += kRootThreads) row[a] = fill;
  __syncthreads();
  if (no_children) return;
  for (int j = tid; j < k; j += kRootThreads) {
    const int64_t c = tb + first + 1 + j;
    const int a = f.actions[c];
    if (a < 0 || a >= A) continue;
    row[a] = tot == 0 ? 1.0 / (double)k : (double)f.visit_counts[c] / (double)tot;
  }
}

// ---- move selection -------------------------------------------------------------------------
// One wavefront per tree.  Temperature 0 takes the first maximum (a wave reduction on
// (value, lowest index)).  Otherwise the lanes compute w = p^(1/T) (w = p for T = 1, 0 for
// p = 0) into LDS, and lane 0 runs the order-dependent part in action order: S = sum of w,
// cdf_a = (w_0/S + ... + w_a/S) / cdf_last, the action is the first a with cdf_a > u.
__global__ __launch_bounds__(kWave) void sample_actions_kernel(omq_forest f, const double* pol,
                                                               double temperature,
                                                               uint64_t seed, uint64_t counter,
                                                               int32_t* actions) {
  extern __shared__ __align__(16) double w[];  // [num_actions]
  const int t = blockIdx.x;
  const int lane = lane_id();
  const int A = f.num_actions;
  const double* p = pol + (int64_t)t * A;
  if (temperature == 0.0) {
    double bv = -1.0;
    int bi = 0x7FFFFFFF;
    for (int a = lane; a < A; a += kWave) {
      const double x = p[a];
      if (x > bv) {  // ascending within the lane: the first maximum of the lane
        bv = x;
        bi = a;
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const double ov = __shfl_xor(bv, off, 64);
      const int oi = __shfl_xor(bi, off, 64);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if (lane == 0) actions[t] = bi;
    return;
  }
  const double inv_t = 1.0 / temperature;
  const bool unit = temperature == 1.0;
  for (int a = lane; a < A; a += kWave) {
    const double x = p[a];
    w[a] = x > 0.0 ? (unit ? x : exp_cw_d(log_cw_d(x) * inv_t)) : 0.0;
  }
  wave_sync();
  double S = 0.0;
  if (lane == 0) {
#pragma unroll 16
    for (int a = 0; a < A; ++a) S = S + w[a];
  }
  S = __shfl(S, 0, 64);
  for (int a = lane; a < A; a += kWave) w[a] = w[a] / S;  // the quotients, once, in parallel
  wave_sync();
  if (lane != 0) return;
  double last = 0.0;
#pragma unroll 16
  for (int a = 0; a < A; ++a) last = last + w[a];
  Stream st = make_stream(seed, counter, t, -1);
  const double u = (double)(splitmix64(st.base) >> 11) * 0x1p-53;  // [0, 1)
  // the first a whose cumulative sum, divided by the total, exceeds u; c / last is monotone
  // in a, so blocks of 16 are skipped while their last cumulative sum stays at or below u
  double c = 0.0;
  int a = 0;
  for (; a + 16 <= A; a += 16) {
    double cb = c;
#pragma unroll
    for (int e = 0; e < 16; ++e) cb = cb + w[a + e];
    if (cb / last > u) break;
    c = cb;
  }
  int pick = A - 1;
  for (; a < A; ++a) {
    c = c + w[a];
    if (c / last > u) {
      pick = a;
      break;
    }
  }
  actions[t] = pick;
}

// ---- root Dirichlet noise -------------------------------------------------------------------
// Entry i of row t is the noise of the i-th legal root action (the layout omq_expand reads).
// The row's legal count L is the root's legal mask popcount (board models) or its sparse-model
// count.  One workgroup per tree: lane-parallel gamma variates, then the canonical wave sum
// and the division.
__global__ __launch_bounds__(kWave) void root_dirichlet_kernel(omq_forest f, double alpha,
                                                               uint64_t seed, uint64_t counter,
                                                               double* noise) {
  const int t = blockIdx.x;
  const int lane = lane_id();
  const int A = f.num_actions;
  double* row = noise + (int64_t)t * A;
  int L;
  if (f.game == OMQ_GAME_SPARSE) {
    L = sparse_legal_count(f, f.root_keys[t]);
  } else {
    int c = 0;
    for (int i = lane; i < f.legal_words; i += kWave)
      c += __popc(f.root_legal[(int64_t)t * f.legal_words + i]);
    L = wave_sum_i(c);
  }
  double part = 0.0;
  for (int i = lane; i < L; i += kWave) {
    Stream st = make_stream(seed, counter, t, i);
    const double g = gamma_mt(alpha, st);
    row[i] = g;
    part = part + g;
  }
  const double S = wave_sum_canonical_d(part);
  for (int i = lane; i < A; i += kWave) {
    if (i < L) row[i] = S > 0.0 ? row[i] / S : 1.0 / (double)L;
    else row[i] = 0.0;
  }
}

// ---- batched Dirichlet noise rows ------------------------------------------------------------
// The reference's batched_dirichlet_noise (mcts_kernels.cu:649-754, host :1735-1790): rows of
// num_actions gamma(alpha, 1) variates divided by their sum (a Dirichlet(alpha, ..., alpha)
// row), left at 0 when the sum is 0.  Entry i of row r is drawn from the stream keyed by
// (seed, counter, r, i); the sum is the canonical wave sum in float64 and each quotient is
// rounded to float32 once.  One wavefront per row.
__global__ __launch_bounds__(kWave) void batched_dirichlet_kernel(int num_actions, double alpha,
                                                                  uint64_t seed,
                                                                  uint64_t counter,
                                                                  float* noise) {
  const int r = blockIdx.x;
  const int lane = lane_id();
  float* row = noise + (int64_t)r * num_actions;
  double part = 0.0;
  for (int i = lane; i < num_actions; i += kWave) {
    Stream st = make_stream(seed, counter, r, i);
    part = part + gamma_mt(alpha, st);
  }
  const double S = wave_sum_canonical_d(part);
  for (int i = lane; i < num_actions; i += kWave) {
    Stream st = make_stream(seed, counter, r, i);  // the same draws again (cheaper than LDS)
    const double g = gamma_mt(alpha, st);
    row[i] = S > 0.0 ? (float)(g / S) : 0.0f;
  }
}

hipError_t launch_batched_dirichlet(int num_sims, int num_actions, double alpha, uint64_t seed,
                                    uint64_t counter, float* noise, hipStream_t st) {
  if (num_sims <= 0 || num_actions <= 0) return hipSuccess;
  hipLaunchKernelGGL(batched_dirichlet_kernel, dim3(num_sims), dim3(kWave), 0, st, num_actions,
                     alpha, seed, counter, noise);
  return hipGetLastError();
}

hipError_t launch_root_policy(const omq_forest& f, double* pol, hipStream_t st) {
  hipLaunchKernelGGL(root_policy_kernel, dim3(f.num_trees), dim3(kRootThreads), 0, st, f, pol);
  return hipGetLastError();
}

hipError_t launch_sample_actions(const omq_forest& f, const double* pol, double temperature,
                                 uint64_t seed, uint64_t counter, int32_t* actions,
                                 hipStream_t st) {
  const size_t lds = (size_t)f.num_actions * sizeof(double);
  hipLaunchKernelGGL(sample_actions_kernel, dim3(f.num_trees), dim3(kWave), lds, st, f, pol,
                     temperature, seed, counter, actions);
  return hipGetLastError();
}

hipError_t launch_root_dirichlet(const omq_forest& f, double alpha, uint64_t seed,
                                 uint64_t counter, double* noise, hipStream_t st) {
  hipLaunchKernelGGL(root_dirichlet_kernel, dim3(f.num_trees), dim3(kWave), 0, st, f, alpha, seed,
                     counter, noise);
  return hipGetLastError();
}

}  // namespace omq
