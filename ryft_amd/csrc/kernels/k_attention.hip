// Fused softmax attention forward for gfx950 (bf16 in, f32 softmax statistics, bf16 P·V, bf16/f32 out).
//
// A workgroup owns 128 queries of one (batch, head); each of its 4 wavefronts owns 32 queries. Key/value blocks of
// 64 rows stream through LDS (double-buffered: block j+1 is fetched while block j is consumed), loaded from global
// memory directly into a swizzled LDS layout without passing through registers. Scores are computed
// transposed, Sᵀ = K·Qᵀ, so that the 32×32 MFMA accumulator puts one query in each lane (lanes l and l+32 share a
// query and split its keys): the running max / sum of the online softmax then need no cross-lane reductions except
// one swap between the two half-waves, and the rescaling of the output Oᵀ = Vᵀ·Pᵀ is a per-lane multiply. P never
// leaves registers: the Sᵀ accumulator, rounded to bf16, is directly the B operand of the P·V MFMA; V stays [key][d]
// in LDS and its transposed fragments, in the matching key order, come from transposing LDS reads. Row maxima are taken on the raw
// scores and each probability costs one FMA and one v_exp_f32 (2^x). Two workgroups share a CU (≤ 256 registers
// per lane), so one wave's softmax overlaps another's MFMAs. The [S, S] score matrix is never materialised.
#include <hip/hip_runtime.h>

#include <string>
#include <type_traits>

#include "../common.h"
#include "ew_device.h"
#include "kernels.h"
#include "launch.h"

namespace ryft {

typedef __bf16 bf16x8_a __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef float f32x16_a __attribute__((__vector_size__(16 * sizeof(float))));
// native 16-byte vector (HIP's uint4 struct copies become memcpys that pin register arrays in private memory)
typedef uint32_t u32x4a __attribute__((ext_vector_type(4)));

bool attention_supported(int head_dim) { return head_dim == 64 || head_dim == 128; }

namespace {

constexpr int BQ = 128;  // queries per workgroup
constexpr int BKV = 64;  // keys per block

__device__ __forceinline__ f32x16_a mma_bf16(const u32x4a& a, const u32x4a& b, f32x16_a c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_a, a), __builtin_bit_cast(bf16x8_a, b), c, 0, 0, 0);
}

typedef uint32_t u32x2a __attribute__((ext_vector_type(2)));
// ds_read_b64_tr_b16 (lane layout measured on gfx950; see the P·V loop) as inline assembly. The compiler sees
// neither its LDS access nor its completion: it does not make it wait for the LDS-DMA loads of the next block (which
// it cannot tell apart from the stage being read, and would otherwise wait for before the first P·V read), and the
// caller waits (lgkmcnt) through tr16_wait before using the result.
template <int OFF>
__device__ __forceinline__ u32x2a lds_read_tr16_asm(uint32_t addr) {
  u32x2a r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}
// waits for all outstanding LDS reads; the fragments pass through the statement so that their uses follow it
__device__ __forceinline__ void tr16_wait(u32x2a (&f)[8]) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5]), "+v"(f[6]), "+v"(f[7]));
}
__device__ __forceinline__ void tr16_wait(u32x2a (&f)[4]) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]));
}

typedef __bf16 bf16x2_a __attribute__((ext_vector_type(2)));
typedef float f32x2_a __attribute__((ext_vector_type(2)));

// Two floats → packed bf16 pair with v_cvt_pk_bf16_f32 (round to nearest even; the values here are finite).
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_a{lo, hi}, bf16x2_a));
}

typedef __attribute__((address_space(3))) void lds_void;
// One wave-wide 16-byte-per-lane load from a buffer straight into LDS: lane l's 16 bytes (buffer bytes voff + soff)
// land at lds + 16·l (lds and soff are wave-uniform: M0 and the scalar offset).
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, char* lds, int voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)lds, 16, voff, soff, 0, 0);
}

template <class F>
__device__ __forceinline__ void static_for4(F&& f) {
  f(std::integral_constant<int, 0>{});
  f(std::integral_constant<int, 1>{});
  f(std::integral_constant<int, 2>{});
  f(std::integral_constant<int, 3>{});
}

template <int D>
struct AttnCfg {
  static constexpr int RB = D * 2;             // bytes per key row of a K or V block in LDS (unpadded, swizzled)
  static constexpr int KBYTES = BKV * RB;      // one K (or V) block
  static constexpr int STAGE = 2 * KBYTES;     // K block, then V block
  static constexpr int PIECES = KBYTES / 1024;  // 1 KB pieces per block: one wave-wide 16-byte-per-lane DMA each
  static constexpr int OP = D * 4 + 16;        // output staging pitch (f32)
  static constexpr int LDS = 2 * STAGE > BQ * OP ? 2 * STAGE : BQ * OP;
};

// LDS swizzle of K and V blocks: the 16-byte chunk c of key row r sits at chunk position c ^ kv_swz(r). Chosen for
// the two read patterns (64 banks of 4 bytes): the K fragment reads (ds_read_b128, 16 lanes on 16 consecutive rows,
// one chunk) need a bijection of r mod 16; the transposing V reads (ds_read_b64_tr_b16, 32 lanes on 4 consecutive
// rows × 4 consecutive chunks) need the 4 rows of a group to land their chunk quads on distinct quads.
template <int D>
__device__ __forceinline__ int kv_swz(int r) {
  if constexpr (D == 128) return ((r & 3) << 2) | ((r >> 2) & 3);  // 16 chunks per row
  else return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);            // 8 chunks per row: bank quad also picks r & 1
}

template <int D>
__global__ void __launch_bounds__(256, 2) attention_fwd_kernel(const AttnArgs A) {
  using C = AttnCfg<D>;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  // Query blocks of 128. Under a causal mask the work of a block grows with its index, so a workgroup takes the
  // blocks p and nq-1-p (the larger first): every workgroup then has the same work. The workgroups of one (batch,
  // head) are consecutive on one XCD (workgroup x runs on XCD x mod 8), so they run together and share that XCD's
  // L2 for the head's keys and values.
  const int nq = A.Sq / BQ;
  const bool pairs = A.causal && nq > 1;
  const int W = pairs ? (nq + 1) / 2 : nq;  // workgroups per (batch, head)
  const int nbh = A.B * A.H;
  int bh, p;
  if (nbh % 8 == 0) {
    const int slot = (int)blockIdx.x >> 3;
    bh = (slot / W) * 8 + ((int)blockIdx.x & 7);
    p = slot % W;
  } else {
    bh = (int)blockIdx.x / W;
    p = (int)blockIdx.x % W;
  }
  const int b = bh / A.H, h = bh % A.H;
  const uint16_t* Qg = (const uint16_t*)A.q + (int64_t)b * A.qs[0] + (int64_t)h * A.qs[1];
  const char* Kg = (const char*)A.k + ((int64_t)b * A.ks[0] + (int64_t)h * A.ks[1]) * 2;
  const char* Vg = (const char*)A.v + ((int64_t)b * A.vs[0] + (int64_t)h * A.vs[1]) * 2;

  // K and V blocks (64 keys × D) go from global memory straight into LDS (buffer_load … lds, 16 bytes per lane):
  // each wave-wide load fills one contiguous 1 KB piece, lane l writing bytes [16l, 16l+16) of it, so the swizzle is
  // applied on the global side — the lane that fills chunk position c' of row r loads chunk c' ^ kv_swz(r). No
  // registers hold the blocks in flight and no LDS stores are issued. The block origin is in the scalar resource
  // and the per-lane byte offsets are loop-invariant (the launcher checks that they fit 32 bits).
  const int ks2 = (int)A.ks[2], vs2 = (int)A.vs[2];
  constexpr int PPW = C::PIECES / 4;  // pieces per wave per tensor
  // the swizzle depends on the row modulo 16 only, which is the same for all pieces of a wave: piece i is piece 0
  // moved down 4096 / RB rows, a scalar offset
  const int r0 = (wave_u * 1024 + lane * 16) / C::RB;
  const int c0 = ((lane * 16) % C::RB / 16) ^ kv_swz<D>(r0);
  const int koff = r0 * ks2 * 2 + c0 * 16, voff = r0 * vs2 * 2 + c0 * 16;
  constexpr int PROWS = 4096 / C::RB;  // rows between a wave's consecutive pieces
  auto dma = [&](int j, int buf) {
    const int k0 = j * BKV;
    const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc((void*)(Kg + (int64_t)k0 * ks2 * 2), (short)0, -1, 0x00020000);
    const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc((void*)(Vg + (int64_t)k0 * vs2 * 2), (short)0, -1, 0x00020000);
    char* sK = smem + buf * C::STAGE;
#pragma unroll
    for (int i = 0; i < PPW; ++i) {
      lds_dma16(kr, sK + (i * 4 + wave_u) * 1024, koff, i * PROWS * ks2 * 2);
      lds_dma16(vr, sK + C::KBYTES + (i * 4 + wave_u) * 1024, voff, i * PROWS * vs2 * 2);
    }
  };
  // wait for this wave's block loads, then for every wave's
  auto dma_wait_sync = [&]() {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
  };

  const int half = lane >> 5;
  // K fragment: row t·32 + l % 32, chunk 2s + l/32 → byte (l % 32)·RB + 16·((2s + l/32) ^ sw) = k_lane ^ 32s
  const int k_lane = (lane & 31) * C::RB + 16 * (kv_swz<D>(lane & 15) ^ half);
  // V fragment rows 16s + vr0 (+ 8), chunk 4·dt + vcl: byte = v_lane[hi] ^ 64·dt, plus 16s·RB
  const int vr0 = 4 * (lane >> 5) + ((lane & 15) >> 2);
  const int vcl = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
  const int v_lo = vr0 * C::RB + 16 * (vcl ^ kv_swz<D>(vr0)) + 8 * (lane & 1);
  const int v_hi = (vr0 + 8) * C::RB + 16 * (vcl ^ kv_swz<D>(vr0 + 8)) + 8 * (lane & 1);

  const float sl2 = A.scale * 1.4426950408889634f;  // logits in the log2 domain
  const int ntiles = pairs && 2 * p + 1 != nq ? 2 : 1;
  for (int ti = 0; ti < ntiles; ++ti) {
    const int qb = pairs ? (ti == 0 ? nq - 1 - p : p) : p;
    const int q0 = qb * BQ;
    // Q fragments (B operand of Sᵀ = K·Qᵀ): lane holds Q[q][s·16 + 8·(lane/32) .. +8] for its query q
    const int myq = q0 + wave * 32 + (lane & 31);
    u32x4a qf[D / 16];
#pragma unroll
    for (int s = 0; s < D / 16; ++s)
      qf[s] = *(const u32x4a*)(Qg + (int64_t)myq * A.qs[2] + s * 16 + 8 * (lane >> 5));
    // complete the Q loads here: waited for at their first use inside the loop, the wait would run every iteration
    // and stall on the next KV block's prefetch (vmcnt(0), expcnt / lgkmcnt left open)
    __builtin_amdgcn_s_waitcnt(0x0F70);
    // Q·scale·log2 e, rounded to bf16 (a relative error of 2^-9 per element, about 1e-3 in a probability): the
    // score MFMAs then yield logits in the log2 domain, and with the accumulator started at -m (the lane's exponent
    // reference) they yield the exponents themselves, so that a probability costs one v_exp_f32 and no FMA
#pragma unroll
    for (int s = 0; s < D / 16; ++s)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t w = qf[s][k];
        qf[s][k] = pack_bf16(__uint_as_float(w << 16) * sl2, __uint_as_float(w & 0xFFFF0000u) * sl2);
      }

    // m_run: the lane's exponent reference in the log2 domain (-inf until its first visible score), cinit its
    // negation (0 while there is none), the score accumulators' start
    float m_run = -INFINITY, l_run = 0.f;
    f32x16_a cinit = f32x16_a{};
    f32x16_a o[D / 32];
#pragma unroll
    for (int t = 0; t < D / 32; ++t) o[t] = f32x16_a{};

    int nkv = A.Sk / BKV;
    if (A.causal) {
      int last_key = q0 + BQ - 1 + A.causal_offset;  // largest key any query of this block may see
      int lim = last_key < 0 ? 0 : last_key / BKV + 1;
      if (lim < nkv) nkv = lim;
    }

    if (nkv > 0) dma(0, 0);
    dma_wait_sync();
    for (int j = 0; j < nkv; ++j) {
      const int cur = j & 1;
      if (j + 1 < nkv) dma(j + 1, cur ^ 1);
      const char* sK = smem + cur * C::STAGE;
      const char* sV = sK + C::KBYTES;
      // Sᵀ tiles: keys [32t, 32t+32) × this wave's 32 queries
      f32x16_a st[2] = {cinit, cinit};
#pragma unroll
      for (int s = 0; s < D / 16; ++s) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          u32x4a kf = *(const u32x4a*)(sK + t * 32 * C::RB + (k_lane ^ (32 * s)));
          st[t] = mma_bf16(kf, qf[s], st[t]);
        }
      }
      // mask and block max on the exponents (logits relative to the reference); only blocks that reach past this
      // wave's first query need the causal mask (a wave-uniform branch between two copies)
      const int kbase = j * BKV;
      const bool need_mask = A.causal && (kbase + BKV - 1 > q0 + wave * 32 + A.causal_offset);
      // The maximum as a signed integer over the exponents' bit patterns: among positive floats the order is the
      // integers' and every negative float (-inf included) is a negative integer, so it tells whether any exponent
      // exceeds 8 — with integer instructions, which run beside the other wave's MFMAs where float ones do not.
      // The float maximum itself is only needed when the reference moves (the rare branch below).
      int imax = (int)0x80000000u;
      if (need_mask) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = kbase + t * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
            const float v = key > myq + A.causal_offset ? -INFINITY : st[t][r];
            st[t][r] = v;
            imax = max(imax, (int)__float_as_uint(v));
          }
      } else {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) imax = max(imax, (int)__float_as_uint(st[t][r]));
      }
      // the other half-wave's maximum, by a lane swap across the halves (no LDS round trip): one of the swap's two
      // results holds it, the other this lane's own value
      auto halves = [](int v) {
        const auto sw = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
        return max(v, max((int)sw[0], (int)sw[1]));
      };
      imax = halves(imax);
      // Lazy rescaling: the exponent reference m_run only moves when this block's maximum exceeds it by more than 8
      // (probabilities then stay ≤ 2^8; o and l share the reference, so o / l is unchanged), and the rescale of o
      // runs only when some lane moved its reference (or has none yet); otherwise P = 2^exponent with no further
      // arithmetic.
      const bool maybe = (imax > (int)0x41000000) | (m_run == -INFINITY);  // 0x41000000 = 8.0f
      u32x4a pf[4];
      // P packed to bf16 (round to nearest even) as the B operand of Oᵀ = Vᵀ·Pᵀ; l sums the packed probabilities
      // (one v_dot2 against (1, 1) per pair), so that o / l weighs V by exactly the probabilities P·V uses
      auto probs = [&]() {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          float p[16];
#pragma unroll
          for (int r = 0; r < 16; ++r) p[r] = __builtin_amdgcn_exp2f(st[t][r]);
          uint32_t w[8];
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            w[k] = pack_bf16(p[2 * k], p[2 * k + 1]);
            l_run = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_a, w[k]),
                                                    __builtin_bit_cast(bf16x2_a, 0x3F803F80u), l_run, false);
          }
          pf[2 * t] = u32x4a{w[0], w[1], w[2], w[3]};
          pf[2 * t + 1] = u32x4a{w[4], w[5], w[6], w[7]};
        }
      };
      if (__builtin_amdgcn_ballot_w64(maybe)) {
        float mloc = -INFINITY;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) mloc = fmaxf(mloc, st[t][r]);
        {
          const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mloc), __float_as_uint(mloc), false, false);
          mloc = fmaxf(mloc, fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])));
        }
        // (bitwise operators: a short-circuit would become a divergent branch)
        const bool raise = (mloc > 8.0f) | ((m_run == -INFINITY) & (mloc != -INFINITY));
        const float shift = raise ? mloc : 0.f;                       // the reference moves up by the block max
        const float m_new = raise ? (m_run == -INFINITY ? 0.f : m_run) + mloc : m_run;
        const float alpha = raise ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.f;  // 0 from a reference of -inf
        l_run *= alpha;
#pragma unroll
        for (int t = 0; t < D / 32; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[t][r] *= alpha;
        m_run = m_new;
        const float c = m_run == -INFINITY ? 0.f : -m_run;
#pragma unroll
        for (int r = 0; r < 16; ++r) cinit[r] = c;
        // this block's exponents relative to the new reference
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) st[t][r] -= shift;
      }
      probs();
      // Oᵀ[d, q] += Σ_key Vᵀ[d, key] · P[q, key]; k-step s covers keys [16s, 16s+16) in the accumulator's key order:
      // element e of lane l ↔ key 16s + 8·(e/4) + 4·(l/32) + e%4. The Vᵀ fragment (row d = l % 32) is read from the
      // [key][d] tile with two ds_read_b64_tr_b16: within each 16-lane group, lane i receives element i % 4 of the
      // 8-byte chunks addressed by lanes i/4 + 4m (m = 0..3), so lane i addresses key row k0 + i/4 and column
      // c0 + 4·(i % 4), and receives keys k0 .. k0+3 of column c0 + i — with k0 = 16s + 4·(l/32) and k0 + 8, exactly
      // the accumulator's key order.
      // Fragments of k-step s + 1 are read while the MFMAs of k-step s run (two register sets).
      const uint32_t vaddr = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const char*)sV;
      u32x2a vf[2][2 * (D / 32)];
      auto vread = [&](auto sc, u32x2a (&f)[2 * (D / 32)]) {
        constexpr int S = decltype(sc)::value;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
          f[2 * dt] = lds_read_tr16_asm<16 * S * C::RB>(vaddr + (v_lo ^ (64 * dt)));
          f[2 * dt + 1] = lds_read_tr16_asm<16 * S * C::RB>(vaddr + (v_hi ^ (64 * dt)));
        }
      };
      vread(std::integral_constant<int, 0>{}, vf[0]);
      static_for4([&](auto sc) {
        constexpr int S = decltype(sc)::value;
        tr16_wait(vf[S & 1]);
        if constexpr (S + 1 < BKV / 16) vread(std::integral_constant<int, S + 1>{}, vf[(S + 1) & 1]);
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
          const u32x2a lo = vf[S & 1][2 * dt], hi = vf[S & 1][2 * dt + 1];
          o[dt] = mma_bf16(u32x4a{lo.x, lo.y, hi.x, hi.y}, pf[S], o[dt]);
        }
      });
      dma_wait_sync();
    }

    // normalise and write out through LDS (lane-per-query layout → row-major rows)
    const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
    const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
    float* so = (float*)smem;
    const int ql = wave * 32 + (lane & 31);
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        int d = dt * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
        *(float*)((char*)so + ql * C::OP + d * 4) = o[dt][r] * inv;
      }
    __syncthreads();
    char* Og = (char*)A.o;
    const int osz = A.out_dtype == DT_F32 ? 4 : 2;
    for (int idx = tid; idx < BQ * D / 4; idx += 256) {
      int qr = idx / (D / 4), c4 = idx % (D / 4);
      float4 v = *(const float4*)((char*)so + qr * C::OP + c4 * 16);
      int64_t off = (int64_t)b * A.os[0] + (int64_t)h * A.os[1] + (int64_t)(q0 + qr) * A.os[2] + c4 * 4;
      if (osz == 4) {
        *(float4*)(Og + off * 4) = v;
      } else {
        uint2 pk = uint2{pack_bf16(v.x, v.y), pack_bf16(v.z, v.w)};
        *(uint2*)(Og + off * 2) = pk;
      }
    }
    __syncthreads();  // the next block's key / value loads reuse the staging area
  }
}

}  // namespace

const char* attention_unsupported(const AttnArgs& a) {
  if (!attention_supported(a.D)) return "attention head dim must be 64 or 128";
  if (a.Sq <= 0 || a.Sk <= 0 || a.Sq % BQ || a.Sk % BKV) return "attention sequence lengths must be multiples of 128 / 64";
  if (a.qs[3] != 1 || a.ks[3] != 1 || a.vs[3] != 1 || a.os[3] != 1)
    return "attention operands must be contiguous along the head dim";
  if (!(a.out_dtype == DT_BF16 || a.out_dtype == DT_F32)) return "attention output type must be bf16 or f32";
  if (a.p_dtype != DT_BF16) return "attention probabilities must be rounded to bf16 before P·V";
  // a row with no visible key (strict mask) is NaN under StableHLO's -inf fill; the kernel does not produce it
  if (a.causal && a.causal_offset < 0) return "attention causal mask must keep the diagonal";
  if (((uintptr_t)a.q | (uintptr_t)a.k | (uintptr_t)a.v | (uintptr_t)a.o) & 15)
    return "attention operands must be 16-byte aligned";
  // Q rows are read 16 bytes at a time, K / V blocks through 32-bit byte offsets from the block origin
  for (int i = 0; i < 3; ++i)
    if ((a.qs[i] | a.ks[i] | a.vs[i] | a.os[i]) & 7) return "attention strides must be multiples of 8 elements";
  if (a.ks[2] > (1 << 20) || a.vs[2] > (1 << 20)) return "attention key/value row stride too large";
  return nullptr;
}

void launch_attention(const AttnArgs& a, hipStream_t stream, hipEvent_t done) {
  if (const char* why = attention_unsupported(a)) fail(PJRT_Error_Code_UNIMPLEMENTED, why);
  // workgroups: per (batch, head), one per query block, or one per pair of blocks under a causal mask
  const int64_t nq = a.Sq / BQ;
  const int64_t blocks = (int64_t)a.B * a.H * (a.causal && nq > 1 ? (nq + 1) / 2 : nq);
  if (blocks == 0) return record_done(done, stream);
  hipError_t e;
  if (a.D == 128) {
    int lds = AttnCfg<128>::LDS;
    static bool attr128 = false;
    if (!attr128) {
      e = hipFuncSetAttribute((const void*)&attention_fwd_kernel<128>, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
      if (e != hipSuccess) fail(PJRT_Error_Code_INTERNAL, std::string("attention LDS attribute: ") + hipGetErrorString(e));
      attr128 = true;
    }
    launch_k(done, attention_fwd_kernel<128>, dim3((unsigned)blocks), dim3(256), (uint32_t)lds, stream, a);
  } else {
    int lds = AttnCfg<64>::LDS;
    static bool attr64 = false;
    if (!attr64) {
      e = hipFuncSetAttribute((const void*)&attention_fwd_kernel<64>, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
      if (e != hipSuccess) fail(PJRT_Error_Code_INTERNAL, std::string("attention LDS attribute: ") + hipGetErrorString(e));
      attr64 = true;
    }
    launch_k(done, attention_fwd_kernel<64>, dim3((unsigned)blocks), dim3(256), (uint32_t)lds, stream, a);
  }
  e = hipGetLastError();
  if (e != hipSuccess) fail(PJRT_Error_Code_INTERNAL, std::string("attention launch failed: ") + hipGetErrorString(e));
}

}  // namespace ryft
