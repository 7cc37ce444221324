// Fused softmax attention forward for gfx950 (bf16 in, f32 softmax statistics, bf16 P·V, bf16/f32 out).
//
// A workgroup owns 128 queries of one (batch, head); each of its 4 wavefronts owns 32 queries. Key/value blocks of
// 64 rows stream through LDS (double-buffered: block j+1 is fetched while block j is consumed). Scores are computed
// transposed, Sᵀ = K·Qᵀ, so that the 32×32 MFMA accumulator puts one query in each lane (lanes l and l+32 share a
// query and split its keys): the running max / sum of the online softmax then need no cross-lane reductions except
// one swap between the two half-waves, and the rescaling of the output Oᵀ = Vᵀ·Pᵀ is a per-lane multiply. P never
// leaves registers: the Sᵀ accumulator, rounded to bf16, is directly the B operand of the P·V MFMA; V stays [key][d]
// in LDS and its transposed fragments, in the matching key order, come from transposing LDS reads. Row maxima are taken on the raw
// scores and each probability costs one FMA and one v_exp_f32 (2^x). Two workgroups share a CU (≤ 256 registers
// per lane), so one wave's softmax overlaps another's MFMAs. The [S, S] score matrix is never materialised.
#include <hip/hip_runtime.h>

#include <string>

#include "../common.h"
#include "ew_device.h"
#include "kernels.h"

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

typedef short s16x4_a __attribute__((ext_vector_type(4)));
// ds_read_b64_tr_b16 (lane layout measured on gfx950; see the P·V loop)
__device__ __forceinline__ uint2 lds_read_tr16(const char* p) {
  const s16x4_a v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4_a*)p);
  return __builtin_bit_cast(uint2, v);
}

typedef __bf16 bf16x2_a __attribute__((ext_vector_type(2)));
typedef float f32x2_a __attribute__((ext_vector_type(2)));

// Two floats → packed bf16 pair with v_cvt_pk_bf16_f32 (round to nearest even; the values here are finite).
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_a{lo, hi}, bf16x2_a));
}

template <int D>
struct AttnCfg {
  static constexpr int KP = D * 2 + 16;  // K row pitch (bytes): [key][d]
  // V row pitch (bytes): [key][d] rows as in memory, ≡ 64 mod 256 so the 4 rows of one transposing read fall in
  // distinct banks
  static constexpr int VP = D * 2 + 64;
  static constexpr int KBYTES = BKV * KP;
  static constexpr int VBYTES = BKV * VP;
  static constexpr int STAGE = KBYTES + VBYTES;
  static constexpr int OP = D * 4 + 16;     // output staging pitch (f32)
  static constexpr int LDS = 2 * STAGE > BQ * OP ? 2 * STAGE : BQ * OP;
};

template <int D>
__global__ void __launch_bounds__(256, 2) attention_fwd_kernel(const AttnArgs A) {
  using C = AttnCfg<D>;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nq = A.Sq / BQ;
  // Under a causal mask the work of a query block grows with its index. Workgroups are dispatched in blockIdx order,
  // so the query block is the slow index and runs heaviest first across all heads (longest-first scheduling): the
  // short blocks fill the tail instead of one head's long blocks finishing last.
  const int nbh = (int)gridDim.x / nq;
  const int qb = A.causal ? nq - 1 - (int)(blockIdx.x / nbh) : (int)(blockIdx.x / nbh);
  const int bh = blockIdx.x % nbh;
  const int b = bh / A.H, h = bh % A.H;
  const int q0 = qb * BQ;
  const uint16_t* Qg = (const uint16_t*)A.q + (int64_t)b * A.qs[0] + (int64_t)h * A.qs[1];
  const char* Kg = (const char*)A.k + ((int64_t)b * A.ks[0] + (int64_t)h * A.ks[1]) * 2;
  const char* Vg = (const char*)A.v + ((int64_t)b * A.vs[0] + (int64_t)h * A.vs[1]) * 2;

  // Q fragments (B operand of Sᵀ = K·Qᵀ): lane holds Q[q][s·16 + 8·(lane/32) .. +8] for its query q
  const int myq = q0 + wave * 32 + (lane & 31);
  u32x4a qf[D / 16];
#pragma unroll
  for (int s = 0; s < D / 16; ++s)
    qf[s] = *(const u32x4a*)(Qg + (int64_t)myq * A.qs[2] + s * 16 + 8 * (lane >> 5));
  // complete the Q loads here: waited for at their first use inside the loop, the wait would run every iteration
  // and stall on the next KV block's prefetch (vmcnt(0), expcnt / lgkmcnt left open)
  __builtin_amdgcn_s_waitcnt(0x0F70);

  const float sl2 = A.scale * 1.4426950408889634f;  // logits in the log2 domain
  float m_run = -INFINITY, l_run = 0.f;
  f32x16_a o[D / 32];
#pragma unroll
  for (int t = 0; t < D / 32; ++t) o[t] = f32x16_a{};

  int nkv = A.Sk / BKV;
  if (A.causal) {
    int last_key = q0 + BQ - 1 + A.causal_offset;  // largest key any query of this block may see
    int lim = last_key < 0 ? 0 : last_key / BKV + 1;
    if (lim < nkv) nkv = lim;
  }

  // K and V blocks (64 keys × D) are copied into LDS unchanged, 16 bytes per thread per load
  constexpr int KVEC = BKV * D / 8 / 256;  // 16-byte vectors of K (and of V) per thread
  u32x4a kreg[KVEC], vreg[KVEC];
  // Buffer loads with the KV block origin in the scalar resource: the per-lane byte offsets are loop-invariant
  // 32-bit values (the launcher checks the extents), so no address registers are rewritten each block — with
  // 64-bit address registers the allocator reuses them while the loads are in flight and the MFMAs then wait for
  // the prefetch.
  const int ks2 = (int)A.ks[2], vs2 = (int)A.vs[2];
  auto gload = [&](int j) {
    const int k0 = j * BKV;
    const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc((void*)(Kg + (int64_t)k0 * ks2 * 2), (short)0, -1, 0x00020000);
    const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc((void*)(Vg + (int64_t)k0 * vs2 * 2), (short)0, -1, 0x00020000);
#pragma unroll
    for (int i = 0; i < KVEC; ++i) {
      int v = tid + i * 256;
      int row = v / (D / 8), c = v % (D / 8);
      kreg[i] = __builtin_amdgcn_raw_buffer_load_b128(kr, (row * ks2 + c * 8) * 2, 0, 0);
      vreg[i] = __builtin_amdgcn_raw_buffer_load_b128(vr, (row * vs2 + c * 8) * 2, 0, 0);
    }
  };
  auto lstore = [&](int buf) {
    char* sK = smem + buf * C::STAGE;
    char* sV = sK + C::KBYTES;
#pragma unroll
    for (int i = 0; i < KVEC; ++i) {
      int v = tid + i * 256;
      int row = v / (D / 8), c = v % (D / 8);
      *(u32x4a*)(sK + row * C::KP + c * 16) = kreg[i];
      *(u32x4a*)(sV + row * C::VP + c * 16) = vreg[i];
    }
  };

  if (nkv > 0) {
    gload(0);
    lstore(0);
  }
  __syncthreads();
  const int half = lane >> 5;
  for (int j = 0; j < nkv; ++j) {
    const int cur = j & 1;
    if (j + 1 < nkv) gload(j + 1);
    const char* sK = smem + cur * C::STAGE;
    const char* sV = sK + C::KBYTES;
    // Sᵀ tiles: keys [32t, 32t+32) × this wave's 32 queries
    f32x16_a st[2] = {f32x16_a{}, f32x16_a{}};
#pragma unroll
    for (int s = 0; s < D / 16; ++s) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        u32x4a kf = *(const u32x4a*)(sK + (t * 32 + (lane & 31)) * C::KP + (s * 16 + 8 * half) * 2);
        st[t] = mma_bf16(kf, qf[s], st[t]);
      }
    }
    // mask and block max on the unscaled scores (the scale is positive, so maxima commute with it); only blocks that
    // reach past this wave's first query need the causal mask (a wave-uniform branch between two copies)
    const int kbase = j * BKV;
    const bool need_mask = A.causal && (kbase + BKV - 1 > q0 + wave * 32 + A.causal_offset);
    float mloc = -INFINITY;
    if (need_mask) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kbase + t * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
          const float v = key > myq + A.causal_offset ? -INFINITY : st[t][r];
          st[t][r] = v;
          mloc = fmaxf(mloc, v);
        }
    } else {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) mloc = fmaxf(mloc, st[t][r]);
    }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
    // Lazy rescaling: the exponent reference m_run only moves when this block's maximum exceeds it by more than 8 in
    // log2 units (probabilities then stay ≤ 2^8; o and l share the reference, so o / l is unchanged), and the
    // rescale of o is skipped when no lane moved its reference.
    const bool raise = (mloc - m_run) * sl2 > 8.0f || (m_run == -INFINITY && mloc != -INFINITY);
    const float m_new = raise ? mloc : m_run;
    const float m_use = m_new == -INFINITY ? 0.f : m_new;  // a fully masked row keeps p = 0
    if (__builtin_amdgcn_ballot_w64(raise)) {
      const float alpha = __builtin_amdgcn_exp2f((m_run - m_use) * sl2);  // 1 where the reference did not move
      l_run *= alpha;
#pragma unroll
      for (int t = 0; t < D / 32; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[t][r] *= alpha;
    }
    m_run = m_new;
    // P = 2^((s - m)·scale·log2 e) with one FMA and v_exp_f32 per score, packed to bf16 (round to nearest even) as
    // the B operand of Oᵀ = Vᵀ·Pᵀ
    const float mb = -m_use * sl2;
    u32x4a pf[4];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      float p[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        p[r] = __builtin_amdgcn_exp2f(fmaf(st[t][r], sl2, mb));
        l_run += p[r];
      }
      pf[2 * t] = u32x4a{pack_bf16(p[0], p[1]), pack_bf16(p[2], p[3]), pack_bf16(p[4], p[5]), pack_bf16(p[6], p[7])};
      pf[2 * t + 1] = u32x4a{pack_bf16(p[8], p[9]), pack_bf16(p[10], p[11]), pack_bf16(p[12], p[13]), pack_bf16(p[14], p[15])};
    }
    // Oᵀ[d, q] += Σ_key Vᵀ[d, key] · P[q, key]; k-step s covers keys [16s, 16s+16) in the accumulator's key order:
    // element e of lane l ↔ key 16s + 8·(e/4) + 4·(l/32) + e%4. The Vᵀ fragment (row d = l % 32) is read from the
    // [key][d] tile with two ds_read_b64_tr_b16: within each 16-lane group, lane i receives element i % 4 of the
    // 8-byte chunks addressed by lanes i/4 + 4m (m = 0..3), so lane i addresses key row k0 + i/4 and column
    // c0 + 4·(i % 4), and receives keys k0 .. k0+3 of column c0 + i — with k0 = 16s + 4·(l/32) and k0 + 8, exactly
    // the accumulator's key order.
    const int v_off = (4 * (lane >> 5) + ((lane & 15) >> 2)) * C::VP + (16 * ((lane >> 4) & 1) + 4 * (lane & 3)) * 2;
#pragma unroll
    for (int s = 0; s < BKV / 16; ++s) {
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt) {
        const char* vp = sV + v_off + 16 * s * C::VP + dt * 64;
        const uint2 lo = lds_read_tr16(vp), hi = lds_read_tr16(vp + 8 * C::VP);
        o[dt] = mma_bf16(u32x4a{lo.x, lo.y, hi.x, hi.y}, pf[s], o[dt]);
      }
    }
    if (j + 1 < nkv) lstore(cur ^ 1);
    __syncthreads();
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
}

}  // namespace

void launch_attention(const AttnArgs& a, hipStream_t stream) {
  if (!attention_supported(a.D)) fail(PJRT_Error_Code_UNIMPLEMENTED, "attention head dim " + std::to_string(a.D));
  if (a.Sq % BQ || a.Sk % BKV) fail(PJRT_Error_Code_UNIMPLEMENTED, "attention sequence lengths must be multiples of 128 / 64");
  if (a.qs[3] != 1 || a.ks[3] != 1 || a.vs[3] != 1 || a.os[3] != 1)
    fail(PJRT_Error_Code_UNIMPLEMENTED, "attention operands must be contiguous along the head dim");
  if (!(a.out_dtype == DT_BF16 || a.out_dtype == DT_F32)) fail(PJRT_Error_Code_UNIMPLEMENTED, "attention output type");
  if (((uintptr_t)a.q | (uintptr_t)a.k | (uintptr_t)a.v | (uintptr_t)a.o) & 15)
    fail(PJRT_Error_Code_UNIMPLEMENTED, "attention operands must be 16-byte aligned");
  // K / V blocks are read through 32-bit byte offsets from the block origin
  if (a.ks[2] > (1 << 20) || a.vs[2] > (1 << 20))
    fail(PJRT_Error_Code_UNIMPLEMENTED, "attention key/value row stride too large");
  int64_t blocks = (int64_t)a.B * a.H * (a.Sq / BQ);
  if (blocks == 0) return;
  hipError_t e;
  if (a.D == 128) {
    int lds = AttnCfg<128>::LDS;
    static bool attr128 = false;
    if (!attr128) {
      e = hipFuncSetAttribute((const void*)&attention_fwd_kernel<128>, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
      if (e != hipSuccess) fail(PJRT_Error_Code_INTERNAL, std::string("attention LDS attribute: ") + hipGetErrorString(e));
      attr128 = true;
    }
    hipLaunchKernelGGL(attention_fwd_kernel<128>, dim3((unsigned)blocks), dim3(256), lds, stream, a);
  } else {
    int lds = AttnCfg<64>::LDS;
    static bool attr64 = false;
    if (!attr64) {
      e = hipFuncSetAttribute((const void*)&attention_fwd_kernel<64>, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
      if (e != hipSuccess) fail(PJRT_Error_Code_INTERNAL, std::string("attention LDS attribute: ") + hipGetErrorString(e));
      attr64 = true;
    }
    hipLaunchKernelGGL(attention_fwd_kernel<64>, dim3((unsigned)blocks), dim3(256), lds, stream, a);
  }
  e = hipGetLastError();
  if (e != hipSuccess) fail(PJRT_Error_Code_INTERNAL, std::string("attention launch failed: ") + hipGetErrorString(e));
}

}  // namespace ryft
