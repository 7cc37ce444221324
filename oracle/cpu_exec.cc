// CPU executor of the five BASELINE graphs and the two HBM calibration graphs: the timed CPU baseline of bench.py (test infrastructure, like the rest of
// oracle/; nothing in the plugin calls it). XLA's CPU PJRT plugin, which ryft-pjrt drives in the reference
// (crates/ryft-pjrt/src/plugins.rs:113-117), cannot be built here, so this stands in for it: each graph of
// ryft_amd/configs.py computed the way an optimising CPU backend runs it — dot_generals as cache-blocked,
// register-tiled GEMMs over packed panels (bf16 / f8E4M3FN operands widened to f32 while packing, as XLA's CPU
// backend upcasts them; int8 with exact int32 accumulation), the elementwise and reduce ops fused into the GEMMs'
// prologues and epilogues, OpenMP across the host's cores. Built with -O3 -march=native -fopenmp (oracle/Makefile;
// bench.py builds it on the host it runs on). tests/test_cpu_exec.py checks every entry point against the numpy
// oracle (oracle/stablehlo.py).
//
// Per-op semantics follow the StableHLO ops the graphs use (ryft-mlir's op docs: dot_general
// linear_algebra.rs:561-705, convert casting.rs:75-122, reduce functional.rs:109-135, logistic / rsqrt
// exponential.rs, multiply / add arithmetic.rs); each op's f32 result is rounded where the graph converts.
#include <omp.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

namespace {

// ------------------------------------------------------------------------------------------------ conversions
inline float bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
inline uint16_t f32_to_bf16(float f) {  // round to nearest even; NaN stays NaN
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
// f8E4M3FN: bias 7, no infinities, 0x7f / 0xff NaN, subnormals m·2^-9
float e4m3_table[256];
struct E4m3Init {
  E4m3Init() {
    for (int v = 0; v < 256; ++v) {
      const int s = v >> 7, e = (v >> 3) & 15, m = v & 7;
      float x;
      if (e == 15 && m == 7) x = NAN;
      else if (e == 0) x = std::ldexp((float)m / 8.0f, -6);
      else x = std::ldexp(1.0f + (float)m / 8.0f, e - 7);
      e4m3_table[v] = s ? -x : x;
    }
  }
} e4m3_init;

// ------------------------------------------------------------------------------------------------ GEMM core
// C[M×N] = A[M×K]·B[K×N] in blocks: for each MC×NC output block (one OpenMP task) and KC slice of K, A and B are
// packed into thread-local panels — A as MR-row strips, k-major; B as NR-column strips, k-major — by the caller's
// loaders (which widen the element type), and an MR×NR register tile of vector accumulators runs over each pair
// of strips. The epilogue functor receives each finished MR×NR tile.
#if defined(__AVX512F__)
constexpr int VW = 16;  // floats per vector register
#else
constexpr int VW = 8;
#endif
typedef float vf __attribute__((vector_size(VW * 4)));
typedef int32_t vi __attribute__((vector_size(VW * 4)));
constexpr int MR = 6, NV = 2, NR = NV * VW;
constexpr int MC = 96, NC = 256, KC = 256;

template <typename T, typename V>
struct Panels {
  std::vector<T> a, b;
  Panels() : a((size_t)MC * KC), b((size_t)KC * NC) {}
};

// One MR×NR tile: acc[i][v] += A strip (k-major, MR per k) × B strip (k-major, NR per k).
template <typename T, typename V>
inline void micro(const T* __restrict a, const T* __restrict b, int kc, V (&acc)[MR][NV]) {
  for (int k = 0; k < kc; ++k) {
    V bv[NV];
    for (int v = 0; v < NV; ++v) std::memcpy(&bv[v], b + (size_t)k * NR + v * VW, sizeof(V));
    for (int i = 0; i < MR; ++i) {
      const T ai = a[(size_t)k * MR + i];
      for (int v = 0; v < NV; ++v) acc[i][v] += ai * bv[v];
    }
  }
}

// T: the arithmetic type (float or int32_t); V its vector. pack_a(m0, mr, k0, kc, dst) writes dst[k*MR + i] (rows
// past mr zero); pack_b(k0, kc, n0, nr, dst) writes dst[k*NR + j] (columns past nr zero); store(m0, mr, n0, nr, acc).
template <typename T, typename V, class PackA, class PackB, class Store>
void gemm(int M, int N, int K, PackA pack_a, PackB pack_b, Store store) {
  const int mb = (M + MC - 1) / MC, nb = (N + NC - 1) / NC;
#pragma omp parallel
  {
    Panels<T, V> p;
#pragma omp for schedule(dynamic, 1) collapse(2)
    for (int bi = 0; bi < mb; ++bi)
      for (int bj = 0; bj < nb; ++bj) {
        const int m0 = bi * MC, n0 = bj * NC;
        const int mcur = std::min(MC, M - m0), ncur = std::min(NC, N - n0);
        const int ms = (mcur + MR - 1) / MR, ns = (ncur + NR - 1) / NR;
        std::vector<V> accs((size_t)ms * ns * MR * NV);
        std::memset(accs.data(), 0, accs.size() * sizeof(V));
        for (int k0 = 0; k0 < K; k0 += KC) {
          const int kc = std::min(KC, K - k0);
          for (int s = 0; s < ms; ++s)
            pack_a(m0 + s * MR, std::min(MR, mcur - s * MR), k0, kc, p.a.data() + (size_t)s * MR * kc);
          for (int t = 0; t < ns; ++t)
            pack_b(k0, kc, n0 + t * NR, std::min(NR, ncur - t * NR), p.b.data() + (size_t)t * NR * kc);
          for (int s = 0; s < ms; ++s)
            for (int t = 0; t < ns; ++t) {
              V(&acc)[MR][NV] = *reinterpret_cast<V(*)[MR][NV]>(accs.data() + ((size_t)s * ns + t) * MR * NV);
              micro<T, V>(p.a.data() + (size_t)s * MR * kc, p.b.data() + (size_t)t * NR * kc, kc, acc);
            }
        }
        for (int s = 0; s < ms; ++s)
          for (int t = 0; t < ns; ++t) {
            const V(&acc)[MR][NV] = *reinterpret_cast<const V(*)[MR][NV]>(accs.data() + ((size_t)s * ns + t) * MR * NV);
            T tile[MR][NR];
            for (int i = 0; i < MR; ++i)
              for (int v = 0; v < NV; ++v) std::memcpy(&tile[i][v * VW], &acc[i][v], sizeof(V));
            store(m0 + s * MR, std::min(MR, mcur - s * MR), n0 + t * NR, std::min(NR, ncur - t * NR), tile);
          }
      }
  }
}

// Loaders for row-major [rows, K] A operands and [K, N] B operands of element type E, widened by `cv`.
template <typename T, typename E, class Cv>
auto rows_a(const E* A, int64_t lda, Cv cv) {
  return [=](int m0, int mr, int k0, int kc, T* dst) {
    for (int k = 0; k < kc; ++k)
      for (int i = 0; i < MR; ++i) dst[(size_t)k * MR + i] = i < mr ? cv(A[(int64_t)(m0 + i) * lda + k0 + k]) : T(0);
  };
}
template <typename T, typename E, class Cv>
auto rows_b(const E* B, int64_t ldb, Cv cv) {
  return [=](int k0, int kc, int n0, int nr, T* dst) {
    for (int k = 0; k < kc; ++k) {
      const E* src = B + (int64_t)(k0 + k) * ldb + n0;
      T* d = dst + (size_t)k * NR;
      for (int j = 0; j < NR; ++j) d[j] = j < nr ? cv(src[j]) : T(0);
    }
  };
}

// f32 → f8E4M3FN, round to nearest even over the 127 finite magnitudes (ascending with their codes); beyond the
// midpoint above the largest finite value (464) and NaN → the NaN code, as the oracle's encode does.
inline uint8_t f32_to_e4m3(float x) {
  const uint8_t sign = std::signbit(x) ? 0x80 : 0;
  const float a = std::fabs(x);
  if (!(a <= 464.0f)) return sign | 0x7f;
  int lo = 0, hi = 126;  // e4m3_table[lo] <= a <= e4m3_table[hi]
  if (a >= e4m3_table[126]) return sign | 0x7e;
  while (hi - lo > 1) {
    const int mid = (lo + hi) / 2;
    if (e4m3_table[mid] <= a) lo = mid;
    else hi = mid;
  }
  const float dl = a - e4m3_table[lo], dh = e4m3_table[hi] - a;
  const int code = dl < dh ? lo : dh < dl ? hi : ((lo & 1) ? hi : lo);
  return sign | (uint8_t)code;
}
// the same encode of every bf16 value, by its bits (a bf16-rounded value is converted with one table load)
uint8_t bf16_e4m3_table[65536];
struct Bf16E4m3Init {
  Bf16E4m3Init() {
    for (int v = 0; v < 65536; ++v) bf16_e4m3_table[v] = f32_to_e4m3(bf16_to_f32((uint16_t)v));
  }
} bf16_e4m3_init;

// rsqrt(Σx²·inv_d + eps) of one bf16 row with the graph's f32 roundings: the squares (exact in f32 for bf16 values)
// summed in double and rounded once, then the f32 multiply, add and rsqrt.
inline float row_rsqrt(const uint16_t* xr, int D, float inv_d, float eps) {
  double ss = 0.0;
  for (int d = 0; d < D; ++d) {
    const float f = bf16_to_f32(xr[d]);
    ss += (double)(f * f);
  }
  const float v = (float)ss * inv_d + eps;
  return (float)(1.0 / std::sqrt((double)v));
}

inline float silu_mul(float g, float u) {  // logistic(g)·g·u in the graph's order: (g·logistic(g))·u
  const float lg = 1.0f / (1.0f + std::exp(-g));
  return (g * lg) * u;
}

}  // namespace

extern "C" {

int cpu_exec_threads() { return omp_get_max_threads(); }

// C1: out[M,N] = a[M,K]·b[K,N], f32.
void cpu_c1(const float* a, const float* b, float* out, int M, int K, int N) {
  auto id = [](float x) { return x; };
  gemm<float, vf>(M, N, K, rows_a<float>(a, K, id), rows_b<float>(b, N, id),
                  [&](int m0, int mr, int n0, int nr, const float (&t)[MR][NR]) {
                    for (int i = 0; i < mr; ++i)
                      for (int j = 0; j < nr; ++j) out[(int64_t)(m0 + i) * N + n0 + j] = t[i][j];
                  });
}

// C2: out[b] = bf16(a[b]·b[b]) for each batch, bf16 operands widened to f32, f32 accumulation.
void cpu_c2(const uint16_t* a, const uint16_t* b, uint16_t* out, int batch, int M, int K, int N) {
  for (int bi = 0; bi < batch; ++bi) {
    const uint16_t* ab = a + (int64_t)bi * M * K;
    const uint16_t* bb = b + (int64_t)bi * K * N;
    uint16_t* ob = out + (int64_t)bi * M * N;
    gemm<float, vf>(M, N, K, rows_a<float>(ab, K, bf16_to_f32), rows_b<float>(bb, N, bf16_to_f32),
                    [&](int m0, int mr, int n0, int nr, const float (&t)[MR][NR]) {
                      for (int i = 0; i < mr; ++i)
                        for (int j = 0; j < nr; ++j) ob[(int64_t)(m0 + i) * N + n0 + j] = f32_to_bf16(t[i][j]);
                    });
  }
}

// C3: acc = a·b (i8 × i8 → i32, exact), out = (f32(acc) · ls[m]) · rs[n].
void cpu_c3(const int8_t* a, const int8_t* b, const float* ls, const float* rs, int32_t* acc, float* out, int M,
            int K, int N) {
  auto wid = [](int8_t x) { return (int32_t)x; };
  gemm<int32_t, vi>(M, N, K, rows_a<int32_t>(a, K, wid), rows_b<int32_t>(b, N, wid),
                    [&](int m0, int mr, int n0, int nr, const int32_t (&t)[MR][NR]) {
                      for (int i = 0; i < mr; ++i)
                        for (int j = 0; j < nr; ++j) {
                          const int64_t o = (int64_t)(m0 + i) * N + n0 + j;
                          acc[o] = t[i][j];
                          out[o] = ((float)t[i][j] * ls[m0 + i]) * rs[n0 + j];
                        }
                    });
}

// C4: causal softmax attention per (batch, head), bf16 q, k, v [B,H,S,D] → bf16 o: s = (q·kᵀ)·scale in f32, keys
// after the query masked (skipped: their probability is exactly 0), f32 softmax (max, exp, sum, divide), the
// probabilities rounded to bf16, o = bf16(p·v) with f32 accumulation. Query blocks of QB rows are the OpenMP tasks;
// each computes its score rows with the GEMM micro-kernel over packed k / v panels.
void cpu_c4(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o, int B, int H, int S, int D,
            float scale) {
  constexpr int QB = 48;  // query rows per task (a multiple of MR)
  constexpr int KB = 128;  // keys per packed v block
  const int nq = (S + QB - 1) / QB;
#pragma omp parallel
  {
    std::vector<float> qa((size_t)QB * D), kb((size_t)D * NR), sc((size_t)QB * S), pa((size_t)KB * MR),
        vb((size_t)KB * NR);
    std::vector<vf> oacc((size_t)(QB / MR) * MR * NV);
#pragma omp for schedule(dynamic, 1) collapse(2)
    for (int bh = 0; bh < B * H; ++bh)
      for (int qi = 0; qi < nq; ++qi) {
        const uint16_t* qh = q + (int64_t)bh * S * D;
        const uint16_t* kh = k + (int64_t)bh * S * D;
        const uint16_t* vh = v + (int64_t)bh * S * D;
        const int q0 = qi * QB, qn = std::min(QB, S - q0), kend = q0 + qn;  // keys [0, kend) are visible to some row
        const int ms = (qn + MR - 1) / MR;
        // A strips of the query block, k-major over D
        for (int s = 0; s < ms; ++s)
          for (int d = 0; d < D; ++d)
            for (int i = 0; i < MR; ++i) {
              const int r = s * MR + i;
              qa[((size_t)s * D + d) * MR + i] = r < qn ? bf16_to_f32(qh[(int64_t)(q0 + r) * D + d]) : 0.0f;
            }
        // scores: key strips of NR keys packed d-major (kᵀ), one MR×NR tile per query strip
        for (int n0 = 0; n0 < kend; n0 += NR) {
          const int nr = std::min(NR, kend - n0);
          for (int d = 0; d < D; ++d)
            for (int j = 0; j < NR; ++j) kb[(size_t)d * NR + j] = j < nr ? bf16_to_f32(kh[(int64_t)(n0 + j) * D + d]) : 0.0f;
          for (int s = 0; s < ms; ++s) {
            vf acc[MR][NV] = {};
            micro<float, vf>(qa.data() + (size_t)s * D * MR, kb.data(), D, acc);
            for (int i = 0; i < MR; ++i) {
              float row[NR];
              for (int w = 0; w < NV; ++w) std::memcpy(&row[w * VW], &acc[i][w], sizeof(vf));
              for (int j = 0; j < nr; ++j) sc[(size_t)(s * MR + i) * S + n0 + j] = row[j] * scale;
            }
          }
        }
        // softmax over the visible keys of each row (k ≤ q), probabilities rounded to bf16
        for (int r = 0; r < qn; ++r) {
          float* srow = sc.data() + (size_t)r * S;
          const int vis = q0 + r + 1;
          float mx = -INFINITY;
          for (int j = 0; j < vis; ++j) mx = std::max(mx, srow[j]);
          float sum = 0.0f;
          for (int j = 0; j < vis; ++j) {
            srow[j] = std::exp(srow[j] - mx);
            sum += srow[j];
          }
          for (int j = 0; j < vis; ++j) srow[j] = bf16_to_f32(f32_to_bf16(srow[j] / sum));
          for (int j = vis; j < kend; ++j) srow[j] = 0.0f;
        }
        // o = p·v over the visible keys: for each NR columns of D, each block of KB keys packs its v rows once
        // (B strip) and every query strip's p (A strip), accumulating per strip
        for (int d0 = 0; d0 < D; d0 += NR) {
          const int dn = std::min(NR, D - d0);
          std::fill(oacc.begin(), oacc.end(), vf{});
          for (int k0 = 0; k0 < kend; k0 += KB) {
            const int kc = std::min(KB, kend - k0);
            for (int kk = 0; kk < kc; ++kk)
              for (int j = 0; j < NR; ++j)
                vb[(size_t)kk * NR + j] = j < dn ? bf16_to_f32(vh[(int64_t)(k0 + kk) * D + d0 + j]) : 0.0f;
            for (int s = 0; s < ms; ++s) {
              for (int kk = 0; kk < kc; ++kk)
                for (int i = 0; i < MR; ++i) {
                  const int r = s * MR + i;
                  pa[(size_t)kk * MR + i] = r < qn ? sc[(size_t)r * S + k0 + kk] : 0.0f;
                }
              vf(&acc)[MR][NV] = *reinterpret_cast<vf(*)[MR][NV]>(oacc.data() + (size_t)s * MR * NV);
              micro<float, vf>(pa.data(), vb.data(), kc, acc);
            }
          }
          for (int s = 0; s < ms; ++s)
            for (int i = 0; i < MR; ++i) {
              const int r = s * MR + i;
              if (r >= qn) break;
              float row[NR];
              for (int w = 0; w < NV; ++w) std::memcpy(&row[w * VW], &oacc[((size_t)s * MR + i) * NV + w], sizeof(vf));
              for (int j = 0; j < dn; ++j) o[((int64_t)bh * S + q0 + r) * D + d0 + j] = f32_to_bf16(row[j]);
            }
        }
      }
  }
}

// C5: SwiGLU MLP with f8E4M3FN weights and per-output-column f32 scales.
//   xn = bf16((x · rsqrt(Σx²/D + eps)) · w)                              (RMSNorm, f32, rounded to bf16)
//   g = (xn·Wg)·sg, u = (xn·Wu)·su, h = bf16((g·logistic(g))·u)           (f8 weights widened exactly)
//   out = bf16((h·Wd)·sd)
void cpu_c5(const uint16_t* x, const uint16_t* w, const uint8_t* wg, const float* sg, const uint8_t* wu,
            const float* su, const uint8_t* wd, const float* sd, uint16_t* out, int M, int D, int F, float inv_d,
            float eps) {
  std::vector<uint16_t> xn((size_t)M * D), h((size_t)M * F);
#pragma omp parallel for schedule(static)
  for (int m = 0; m < M; ++m) {
    const float r = row_rsqrt(x + (int64_t)m * D, D, inv_d, eps);
    const uint16_t* xr = x + (int64_t)m * D;
    for (int d = 0; d < D; ++d) xn[(size_t)m * D + d] = f32_to_bf16((bf16_to_f32(xr[d]) * r) * bf16_to_f32(w[d]));
  }
  auto f8 = [](uint8_t b) { return e4m3_table[b]; };
  // gate and up as one GEMM over the interleaved columns [g_n0 .. g_n0+NR/2) | [u_n0 .. ): each NR-wide B strip
  // holds NR/2 gate and NR/2 up columns, so the epilogue sees both for the same output columns
  constexpr int HN = NR / 2;
  gemm<float, vf>(
      M, 2 * F, D, rows_a<float>(xn.data(), D, bf16_to_f32),
      [&](int k0, int kc, int n0, int nr, float* dst) {
        const int c0 = n0 / 2;  // n0 is a multiple of NR: output columns [c0, c0 + HN)
        const int cn = nr / 2;
        for (int k = 0; k < kc; ++k) {
          const uint8_t* gr = wg + (int64_t)(k0 + k) * F + c0;
          const uint8_t* ur = wu + (int64_t)(k0 + k) * F + c0;
          float* d = dst + (size_t)k * NR;
          for (int j = 0; j < HN; ++j) {
            d[j] = j < cn ? f8(gr[j]) : 0.0f;
            d[HN + j] = j < cn ? f8(ur[j]) : 0.0f;
          }
        }
      },
      [&](int m0, int mr, int n0, int nr, const float (&t)[MR][NR]) {
        const int c0 = n0 / 2, cn = nr / 2;
        for (int i = 0; i < mr; ++i)
          for (int j = 0; j < cn; ++j) {
            const float g = t[i][j] * sg[c0 + j], u = t[i][HN + j] * su[c0 + j];
            h[(size_t)(m0 + i) * F + c0 + j] = f32_to_bf16(silu_mul(g, u));
          }
      });
  gemm<float, vf>(M, D, F, rows_a<float>(h.data(), F, bf16_to_f32), rows_b<float>(wd, D, f8),
                  [&](int m0, int mr, int n0, int nr, const float (&t)[MR][NR]) {
                    for (int i = 0; i < mr; ++i)
                      for (int j = 0; j < nr; ++j)
                        out[(int64_t)(m0 + i) * D + n0 + j] = f32_to_bf16(t[i][j] * sd[n0 + j]);
                  });
}

// The HBM copy calibration: y = -x over n f32 values.
void cpu_copy_negate(const float* x, float* y, int64_t n) {
#pragma omp parallel for simd schedule(static)
  for (int64_t i = 0; i < n; ++i) y[i] = -x[i];
}

// The RMSNorm calibration: out = f8E4M3FN(bf16((x · rsqrt(Σx²/D + eps)) · w)) per row of D bf16 values.
void cpu_rmsnorm_f8(const uint16_t* x, const uint16_t* w, uint8_t* out, int M, int D, float inv_d, float eps) {
#pragma omp parallel for schedule(static)
  for (int m = 0; m < M; ++m) {
    const uint16_t* xr = x + (int64_t)m * D;
    const float r = row_rsqrt(xr, D, inv_d, eps);
    for (int d = 0; d < D; ++d)
      out[(int64_t)m * D + d] = bf16_e4m3_table[f32_to_bf16((bf16_to_f32(xr[d]) * r) * bf16_to_f32(w[d]))];
  }
}

}  // extern "C"
