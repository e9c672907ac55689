// A non-Python caller of libint8kv.so: only the extern "C" entry points of include/int8kv.h and the
// HIP runtime, no torch.  It writes bf16 K/V of three sequences into paged INT8 caches
// (int8kv_cache_write), decodes one query token per sequence (int8kv_paged_decode, automatic and
// forced-split layouts, and int8kv_paged_decode_noalloc) and checks, on the CPU:
//   - every cache byte equals clamp(rint(x / s), -127, 127) with an IEEE fp32 quotient, rounded
//     half to even (src/quant.py:37-40), and unwritten slots keep their fill byte;
//   - the outputs against softmax attention recomputed in double precision from those int8 codes
//     (max |diff| <= 2e-2 and cosine >= 0.9999, the output being bf16);
//   - the no-allocation entry point returns the same bytes as the workspace one.
// Exit status 0 when every check passes.  Arguments: none (fixed seed).

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <utility>
#include <vector>

#include "int8kv.h"

namespace {

constexpr int kHq = 28, kHkv = 4, kD = 128, kBS = 16, kFill = 0x5A;

#define HIP_OK(x)                                                            \
  do {                                                                       \
    hipError_t e_ = (x);                                                     \
    if (e_ != hipSuccess) {                                                  \
      std::fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorString(e_));    \
      std::exit(2);                                                          \
    }                                                                        \
  } while (0)

#define LIB_OK(x)                                              \
  do {                                                         \
    int s_ = (x);                                              \
    if (s_ != INT8KV_OK) {                                     \
      std::fprintf(stderr, "%s returned %d\n", #x, s_);        \
      std::exit(3);                                            \
    }                                                          \
  } while (0)

uint64_t g_state = 0x9E3779B97F4A7C15ull;
double uniform() {  // xorshift64*, in [0, 1)
  g_state ^= g_state >> 12;
  g_state ^= g_state << 25;
  g_state ^= g_state >> 27;
  return (double)((g_state * 0x2545F4914F6CDD1Dull) >> 11) * (1.0 / 9007199254740992.0);
}
double normal() {
  const double u = uniform() + 1e-12, v = uniform();
  return std::sqrt(-2.0 * std::log(u)) * std::cos(6.283185307179586 * v);
}

uint16_t to_bf16(float f) {  // round to nearest even
  uint32_t u;
  std::memcpy(&u, &f, 4);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
float from_bf16(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

template <typename T>
T* device_copy(const std::vector<T>& v) {
  T* p = nullptr;
  HIP_OK(hipMalloc(&p, v.size() * sizeof(T)));
  HIP_OK(hipMemcpy(p, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice));
  return p;
}

}  // namespace

int main() {
  const std::vector<int32_t> lens = {1, 37, 300};
  const int B = (int)lens.size();
  int blocks_needed = 0, width = 0;
  for (int L : lens) {
    blocks_needed += (L + kBS - 1) / kBS;
    width = std::max(width, (L + kBS - 1) / kBS);
  }
  const int NB = blocks_needed + 5;
  // Block table: sequences take distinct blocks of a shuffled pool.
  std::vector<int32_t> pool(NB);
  for (int i = 0; i < NB; ++i) pool[i] = i;
  for (int i = NB - 1; i > 0; --i) std::swap(pool[i], pool[(int)(uniform() * (i + 1))]);
  std::vector<int32_t> table((size_t)B * width, 0);
  std::vector<int64_t> slots;
  int next = 0;
  for (int b = 0; b < B; ++b)
    for (int t = 0; t < lens[b]; ++t) {
      if (t % kBS == 0) table[(size_t)b * width + t / kBS] = pool[next++];
      slots.push_back((int64_t)table[(size_t)b * width + t / kBS] * kBS + t % kBS);
    }
  const int T = (int)slots.size();

  // bf16 K/V [T, Hkv, D] (K with a few large channels), query [B, Hq, D]; scales absmax / 127.
  std::vector<uint16_t> k((size_t)T * kHkv * kD), v(k.size()), q((size_t)B * kHq * kD);
  for (size_t i = 0; i < k.size(); ++i) {
    const int ch = (int)(i % kD);
    k[i] = to_bf16((float)(normal() * (ch % 37 == 3 ? 8.0 : 1.0)));
    v[i] = to_bf16((float)(normal() * 0.5));
  }
  for (auto& x : q) x = to_bf16((float)normal());
  std::vector<float> ks(kHkv, 0.0f), vs(kHkv, 0.0f);
  for (int t = 0; t < T; ++t)
    for (int h = 0; h < kHkv; ++h)
      for (int d = 0; d < kD; ++d) {
        const size_t i = ((size_t)t * kHkv + h) * kD + d;
        ks[h] = std::max(ks[h], std::fabs(from_bf16(k[i])));
        vs[h] = std::max(vs[h], std::fabs(from_bf16(v[i])));
      }
  for (int h = 0; h < kHkv; ++h) {
    ks[h] = std::max(ks[h] / 127.0f, 1e-6f);
    vs[h] = std::max(vs[h] / 127.0f, 1e-6f);
  }

  const size_t cache_bytes = (size_t)NB * kBS * kHkv * kD;
  std::vector<int8_t> fill(cache_bytes, (int8_t)kFill);
  uint16_t* dk = device_copy(k);
  uint16_t* dv = device_copy(v);
  uint16_t* dq = device_copy(q);
  int8_t* dkc = device_copy(fill);
  int8_t* dvc = device_copy(fill);
  int64_t* dslots = device_copy(slots);
  int32_t* dtable = device_copy(table);
  int32_t* dlens = device_copy(lens);
  float* dks = device_copy(ks);
  float* dvs = device_copy(vs);
  uint16_t *dout = nullptr, *dout2 = nullptr, *dout3 = nullptr;
  HIP_OK(hipMalloc(&dout, q.size() * 2));
  HIP_OK(hipMalloc(&dout2, q.size() * 2));
  HIP_OK(hipMalloc(&dout3, q.size() * 2));
  hipStream_t stream;
  HIP_OK(hipStreamCreate(&stream));

  const int64_t src_st[3] = {kHkv * kD, kD, 1};
  const int64_t cache_st[4] = {kBS * kHkv * kD, kHkv * kD, kD, 1};
  const int64_t q_st[3] = {kHq * kD, kD, 1};
  const int64_t t_st[2] = {width, 1};
  LIB_OK(int8kv_cache_write(dk, dv, INT8KV_BF16, T, kHkv, kD, src_st, src_st, dkc, dvc, NB, kBS,
                            cache_st, cache_st, dslots, INT8KV_I64, dks, dvs, stream));
  const size_t ws_bytes = int8kv_decode_workspace_bytes(kHq, kHkv, kD, kBS, 0);
  const size_t ws3_bytes = int8kv_decode_workspace_bytes(kHq, kHkv, kD, kBS, 3 * B);
  void *ws = nullptr, *ws3 = nullptr;
  HIP_OK(hipMalloc(&ws, ws_bytes));
  HIP_OK(hipMalloc(&ws3, ws3_bytes));
  const float sm = 1.0f / std::sqrt((float)kD);
  LIB_OK(int8kv_paged_decode(dq, INT8KV_BF16, B, kHq, kD, q_st, dkc, dvc, INT8KV_I8, NB, kBS, kHkv,
                             cache_st, cache_st, dtable, INT8KV_I32, width, t_st, dlens, INT8KV_I32,
                             dks, dvs, sm, dout, q_st, ws, ws_bytes, 0, 0, INT8KV_DECODE_ALL,
                             stream));
  LIB_OK(int8kv_paged_decode(dq, INT8KV_BF16, B, kHq, kD, q_st, dkc, dvc, INT8KV_I8, NB, kBS, kHkv,
                             cache_st, cache_st, dtable, INT8KV_I32, width, t_st, dlens, INT8KV_I32,
                             dks, dvs, sm, dout3, q_st, ws3, ws3_bytes, 3 * B, 2,
                             INT8KV_DECODE_ALL, stream));
  LIB_OK(int8kv_paged_decode_noalloc(dq, INT8KV_BF16, B, kHq, kD, q_st, dkc, dvc, INT8KV_I8, NB,
                                     kBS, kHkv, cache_st, cache_st, dtable, INT8KV_I32, width,
                                     t_st, dlens, INT8KV_I32, dks, dvs, sm, dout2, q_st, 0, 0,
                                     INT8KV_DECODE_ALL, stream));
  HIP_OK(hipStreamSynchronize(stream));
  int8kv_decode_plan_t plan;
  LIB_OK(int8kv_decode_plan(INT8KV_BF16, INT8KV_I8, B, kHq, kHkv, kD, NB, kBS, width, kD, kD, 0, 0,
                            INT8KV_DECODE_ALL, 0, 0, &plan));
  std::printf("automatic plan: layout %d, %d kernel(s), %d ranges, workspace %llu bytes\n",
              plan.layout, plan.kernels, plan.num_ranges,
              (unsigned long long)plan.workspace_bytes);

  std::vector<int8_t> kc(cache_bytes), vc(cache_bytes);
  std::vector<uint16_t> out(q.size()), out2(q.size()), out3(q.size());
  HIP_OK(hipMemcpy(kc.data(), dkc, cache_bytes, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(vc.data(), dvc, cache_bytes, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(out.data(), dout, out.size() * 2, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(out2.data(), dout2, out.size() * 2, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(out3.data(), dout3, out.size() * 2, hipMemcpyDeviceToHost));

  // 1. Cache bytes: every written slot as the quantisation gives it, every other byte the fill.
  std::vector<int8_t> want_k(cache_bytes, (int8_t)kFill), want_v(cache_bytes, (int8_t)kFill);
  for (int t = 0; t < T; ++t)
    for (int h = 0; h < kHkv; ++h)
      for (int d = 0; d < kD; ++d) {
        const size_t src = ((size_t)t * kHkv + h) * kD + d;
        const size_t dst = ((size_t)slots[t] * kHkv + h) * kD + d;
        const float qk = from_bf16(k[src]) / ks[h];  // IEEE fp32 quotient
        const float qv = from_bf16(v[src]) / vs[h];
        want_k[dst] = (int8_t)std::fmin(std::fmax(std::rint(qk), -127.0f), 127.0f);
        want_v[dst] = (int8_t)std::fmin(std::fmax(std::rint(qv), -127.0f), 127.0f);
      }
  size_t bad = 0;
  for (size_t i = 0; i < cache_bytes; ++i) bad += (kc[i] != want_k[i]) + (vc[i] != want_v[i]);
  std::printf("cache bytes differing from the quantisation: %zu of %zu\n", bad, 2 * cache_bytes);

  // 2. Attention from the int8 codes in double precision.
  const int G = kHq / kHkv;
  double max_abs = 0.0, dot = 0.0, n_got = 0.0, n_ref = 0.0, max_abs3 = 0.0;
  std::vector<double> s;
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < kHq; ++h) {
      const int g = h / G;
      const int L = lens[b];
      s.assign(L, 0.0);
      double m = -1e300;
      for (int t = 0; t < L; ++t) {
        const int64_t slot = (int64_t)table[(size_t)b * width + t / kBS] * kBS + t % kBS;
        double acc = 0.0;
        for (int d = 0; d < kD; ++d)
          acc += (double)from_bf16(q[((size_t)b * kHq + h) * kD + d]) *
                 kc[((size_t)slot * kHkv + g) * kD + d];
        s[t] = acc * ks[g] * sm;
        m = std::max(m, s[t]);
      }
      double l = 0.0;
      for (int t = 0; t < L; ++t) l += (s[t] = std::exp(s[t] - m));
      for (int d = 0; d < kD; ++d) {
        double o = 0.0;
        for (int t = 0; t < L; ++t) {
          const int64_t slot = (int64_t)table[(size_t)b * width + t / kBS] * kBS + t % kBS;
          o += s[t] * vc[((size_t)slot * kHkv + g) * kD + d];
        }
        o = o / l * vs[g];
        const size_t i = ((size_t)b * kHq + h) * kD + d;
        const double got = from_bf16(out[i]);
        max_abs = std::max(max_abs, std::fabs(got - o));
        max_abs3 = std::max(max_abs3, std::fabs((double)from_bf16(out3[i]) - o));
        dot += got * o;
        n_got += got * got;
        n_ref += o * o;
      }
    }
  const double cosine = dot / std::sqrt(n_got * n_ref);
  std::printf("decode vs double-precision reference: max|diff| %.3e (forced splits %.3e), cos %.7f\n",
              max_abs, max_abs3, cosine);

  // 3. The no-allocation entry point gives the same bytes.
  const bool same = std::memcmp(out.data(), out2.data(), out.size() * 2) == 0;
  std::printf("noalloc output identical: %s\n%s\n", same ? "yes" : "no", int8kv_version());

  const bool ok = bad == 0 && max_abs <= 2e-2 && max_abs3 <= 2e-2 && cosine >= 0.9999 && same;
  std::printf("%s\n", ok ? "ABI SMOKE OK" : "ABI SMOKE FAILED");
  return ok ? 0 : 1;
}
