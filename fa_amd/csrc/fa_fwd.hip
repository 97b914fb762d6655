// Flash-attention forward for MI355X (gfx950): non-causal GQA, D = 128,
// FP16 in/out, FP32- or FP16-accumulated O.
//
// Work decomposition (reference: task = (batch*head, query block), KV head
// = head / group, backends/cce_fa_nk_nz_vector_fp32_v5_sumpack/project/
// op_kernel/panel_kernel.h:264-274): one workgroup owns BM = NW*SUB*32 query
// rows of one (batch, head); each wave owns SUB subtiles of 32 rows. The
// workgroup streams the whole key range in blocks of BN keys; each K block
// and V^T block is staged once in LDS (double-buffered) and read by every
// wave, and every wave keeps its Q fragments, O accumulators and softmax
// statistics in registers for the whole key loop.
//
// Matrix products run transposed so the softmax is lane-local:
//   S^T = K Q^T   v_mfma_f32_32x32x16_f16, A = K rows from LDS, B = Q^T
//                 from registers. Lane l holds query row l%32 and 16 keys
//                 per 32x32 tile.
//   O^T += V^T P^T  A = V^T rows from LDS, B = P^T straight from the S^T
//                 registers (converted to FP16). Lane l keeps query row l%32
//                 for all its O registers, so rescaling by alpha is per lane.
// The 32x32 output layout gives a lane keys {8g+4h .. 8g+4h+3} (g = 0..3,
// h = lane/32); the PV step over keys 16s..16s+15 therefore wants, in its k
// slots 8h..8h+7, keys {16s+4h..+3, 16s+8+4h..+3}. The V transpose kernel
// writes V^T with exactly that key order inside every 16-key group, so each
// A fragment is one 16-byte LDS read.
//
// Online softmax in base 2 with the scale folded in (c = scale*log2(e)):
//   m' = max(m, rowmax(S)),  alpha = 2^((m - m') c),  P = 2^(S c - m' c),
//   l' = alpha l + rowsum(P16),  O' = alpha O + P16 V
// where P16 is P rounded to FP16 (the MFMA operand) and the row sum is taken
// over the same rounded values, so numerator and denominator use identical
// weights. Semantics follow the reference's FP32 vector softmax
// (project/op_kernel/online_softmax.h:86-224, vector_output.h:22-86 of the
// FP32 variant) and, for FA_ACC_FP16, its FP16-O merge (vector_output.h:
// 130-210 of backends/cce_fa_nqkq_nz_resident_v13_q768_pool_i4_p128).

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>

#include "../../include/fa_hip.h"

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int HD = 128;               // head dimension
constexpr int VT_GROUP = 64;          // keys per V-transpose workgroup
constexpr float NEG_BIG = -1.0e30f;   // finite "minus infinity" for the running max
constexpr double LOG2E = 1.4426950408889634;

// 16-byte chunk swizzle for an LDS tile whose rows are CPR chunks long.
// Rows are read 32 at a time at one logical chunk column; the XOR spreads any
// 16 consecutive rows over 16 distinct 16-byte bank groups (256 bytes).
template <int CPR>
__device__ __forceinline__ int swz(int row, int chunk) {
  constexpr int RPW = 16 / CPR;       // rows sharing one 256-byte bank window
  return chunk ^ ((row / RPW) & (CPR - 1));
}

// Combine a per-lane value with the lane 32 apart (same query row, other
// half of the keys).
__device__ __forceinline__ float half_max(float x) {
  auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float half_sum(float x) {
  auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

__device__ __forceinline__ f32x16 mfma32(h8 a, h8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Key slot -> key inside a 16-key group of the transposed V (see header).
__device__ __forceinline__ int vt_key_of_slot(int slot) {
  const int h = slot >> 3, e = slot & 7;
  return (e < 4) ? (4 * h + e) : (8 + 4 * h + (e - 4));
}

// vt[kv][d][key0 + slot] = v[kv][key0 + key(slot)][d], one 64-key group per
// workgroup. Grid (Nk / 64, B * Hkv), 256 threads.
__global__ void __launch_bounds__(256) fa_vt_kernel(const _Float16* __restrict__ v,
                                                    _Float16* __restrict__ vt, int seq_k) {
  __shared__ _Float16 tile[VT_GROUP][HD + 8];
  const int tid = threadIdx.x;
  const size_t kv = blockIdx.y;
  const int key0 = blockIdx.x * VT_GROUP;
  const _Float16* src = v + (kv * seq_k + key0) * HD;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = tid + 256 * j;
    const int r = i >> 4, ch = i & 15;
    *reinterpret_cast<u32x4*>(&tile[r][ch * 8]) =
        *reinterpret_cast<const u32x4*>(src + (size_t)r * HD + ch * 8);
  }
  __syncthreads();
  _Float16* dst = vt + kv * HD * (size_t)seq_k + key0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = tid + 256 * j;
    const int d = i >> 3, ch = i & 7;
    h8 val;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int slot = (ch & 1) * 8 + e;
      val[e] = tile[16 * (ch >> 1) + vt_key_of_slot(slot)][d];
    }
    *reinterpret_cast<h8*>(dst + (size_t)d * seq_k + ch * 8) = val;
  }
}

// The attention body. ACC16 selects the FP16 O accumulator; NW waves per
// workgroup, SUB 32-row subtiles per wave, BN keys per block.
template <bool ACC16, int NW, int SUB, int BN>
__device__ __forceinline__ void fa_fwd_body(const _Float16* __restrict__ q,
                                            const _Float16* __restrict__ k,
                                            const _Float16* __restrict__ vt,
                                            _Float16* __restrict__ o, int heads_q, int group,
                                            int seq_q, int seq_k, float c) {
  constexpr int NT = NW * 64;
  constexpr int BM = NW * SUB * 32;
  constexpr int KT = BN / 32;          // 32-key S^T tiles per block
  constexpr int KS = BN / 16;          // 16-key PV steps per block
  constexpr int KCH = BN * 16;         // 16-byte chunks in a K block (BN rows x 256 B)
  constexpr int VCPR = BN / 8;         // chunks per V^T row (BN keys)
  constexpr int VCH = HD * VCPR;       // chunks in a V^T block
  constexpr int KLD = KCH / NT;        // K chunks each thread stages per block
  constexpr int VLD = VCH / NT;
  static_assert(KCH % NT == 0 && VCH % NT == 0, "block must split evenly over threads");
  static_assert(BN % 32 == 0, "BN must be a multiple of 32");

  __shared__ u32x4 smem[2][KCH + VCH];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hf = lane >> 5;

  const int tiles_q = seq_q / BM;
  const int bh = blockIdx.x / tiles_q;
  const int qt = blockIdx.x - bh * tiles_q;
  const int b = bh / heads_q, h = bh - b * heads_q;
  const int heads_kv = heads_q / group;
  const size_t kv = (size_t)b * heads_kv + h / group;
  const _Float16* kp = k + kv * (size_t)seq_k * HD;
  const _Float16* vp = vt + kv * (size_t)HD * seq_k;
  const size_t row0 = (size_t)bh * seq_q + (size_t)qt * BM + (size_t)wave * (SUB * 32);
  const _Float16* qp = q + row0 * HD;
  _Float16* op = o + row0 * HD;

  // Q^T operand fragments: lane holds query row l32, dims 16kk+8hf..+7.
  h8 qf[SUB][8];
#pragma unroll
  for (int u = 0; u < SUB; ++u)
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
      qf[u][kk] = *reinterpret_cast<const h8*>(qp + (size_t)(u * 32 + l32) * HD + kk * 16 + hf * 8);

  u32x4 kreg[KLD], vreg[VLD];
  auto gload = [&](int blk) {
    const int key0 = blk * BN;
#pragma unroll
    for (int j = 0; j < KLD; ++j) {
      const int i = tid + j * NT;
      const int r = i >> 4, ch = i & 15;
      kreg[j] = *reinterpret_cast<const u32x4*>(kp + (size_t)(key0 + r) * HD + ch * 8);
    }
#pragma unroll
    for (int j = 0; j < VLD; ++j) {
      const int i = tid + j * NT;
      const int d = i / VCPR, ch = i % VCPR;
      vreg[j] = *reinterpret_cast<const u32x4*>(vp + (size_t)d * seq_k + key0 + ch * 8);
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int j = 0; j < KLD; ++j) {
      const int i = tid + j * NT;
      const int r = i >> 4, ch = i & 15;
      smem[buf][r * 16 + swz<16>(r, ch)] = kreg[j];
    }
#pragma unroll
    for (int j = 0; j < VLD; ++j) {
      const int i = tid + j * NT;
      const int d = i / VCPR, ch = i % VCPR;
      smem[buf][KCH + d * VCPR + swz<VCPR>(d, ch)] = vreg[j];
    }
  };

  f32x16 acc[SUB][4];                  // FP32 O^T: dims 32dt.., queries l32
  h2 acc16[SUB][4][8];                 // FP16 O^T, same element order, packed in pairs
  float m[SUB], lsum[SUB];
#pragma unroll
  for (int u = 0; u < SUB; ++u) {
    m[u] = NEG_BIG;
    lsum[u] = 0.f;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      if constexpr (ACC16) {
#pragma unroll
        for (int i = 0; i < 8; ++i) acc16[u][dt][i] = h2{(_Float16)0.f, (_Float16)0.f};
      } else {
        acc[u][dt] = f32x16{};
      }
    }
  }
  const h2 ones = {(_Float16)1.f, (_Float16)1.f};

  gload(0);
  lstore(0);
  __syncthreads();

  const int nblk = seq_k / BN;
  for (int n = 0; n < nblk; ++n) {
    const int buf = n & 1;
    if (n + 1 < nblk) gload(n + 1);
    const u32x4* kb = smem[buf];
    const u32x4* vb = smem[buf] + KCH;

    // S^T = K Q^T
    f32x16 s[SUB][KT];
#pragma unroll
    for (int u = 0; u < SUB; ++u)
#pragma unroll
      for (int t = 0; t < KT; ++t) s[u][t] = f32x16{};
#pragma unroll
    for (int t = 0; t < KT; ++t) {
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const int r = t * 32 + l32;
        const h8 a = __builtin_bit_cast(h8, kb[r * 16 + swz<16>(r, 2 * kk + hf)]);
#pragma unroll
        for (int u = 0; u < SUB; ++u) s[u][t] = mfma32(a, qf[u][kk], s[u][t]);
      }
    }

    // Online softmax, one query row per lane pair.
    h8 p[SUB][KS];
    float alpha[SUB];
#pragma unroll
    for (int u = 0; u < SUB; ++u) {
      float mx = s[u][0][0];
#pragma unroll
      for (int t = 0; t < KT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[u][t][r]);
      mx = half_max(mx);
      const float mnew = fmaxf(m[u], mx);
      alpha[u] = __builtin_amdgcn_exp2f((m[u] - mnew) * c);
      m[u] = mnew;
      const float mc = mnew * c;
      float ls = 0.f;
#pragma unroll
      for (int t = 0; t < KT; ++t) {
#pragma unroll
        for (int g2 = 0; g2 < 2; ++g2) {
          h8 frag;
#pragma unroll
          for (int e = 0; e < 8; e += 2) {
            const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[u][t][8 * g2 + e], c, -mc));
            const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[u][t][8 * g2 + e + 1], c, -mc));
            const h2 pr = {(_Float16)p0, (_Float16)p1};
            frag[e] = pr[0];
            frag[e + 1] = pr[1];
            ls = __builtin_amdgcn_fdot2(pr, ones, ls, false);
          }
          p[u][2 * t + g2] = frag;
        }
      }
      lsum[u] = lsum[u] * alpha[u] + ls;
      if constexpr (!ACC16) {
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) acc[u][dt] *= alpha[u];
      }
    }

    // O^T += V^T P^T
    if constexpr (!ACC16) {
#pragma unroll
      for (int st = 0; st < KS; ++st) {
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          const int r = dt * 32 + l32;
          const h8 a = __builtin_bit_cast(h8, vb[r * VCPR + swz<VCPR>(r, 2 * st + hf)]);
#pragma unroll
          for (int u = 0; u < SUB; ++u) acc[u][dt] = mfma32(a, p[u][st], acc[u][dt]);
        }
      }
    } else {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        f32x16 part[SUB];
#pragma unroll
        for (int u = 0; u < SUB; ++u) part[u] = f32x16{};
#pragma unroll
        for (int st = 0; st < KS; ++st) {
          const int r = dt * 32 + l32;
          const h8 a = __builtin_bit_cast(h8, vb[r * VCPR + swz<VCPR>(r, 2 * st + hf)]);
#pragma unroll
          for (int u = 0; u < SUB; ++u) part[u] = mfma32(a, p[u][st], part[u]);
        }
        // O16 = alpha * O16 + fp16(partial), the FP16-O merge.
#pragma unroll
        for (int u = 0; u < SUB; ++u) {
          const _Float16 a16 = (_Float16)alpha[u];
          const h2 a2 = {a16, a16};
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const h2 pv = {(_Float16)part[u][2 * i], (_Float16)part[u][2 * i + 1]};
            acc16[u][dt][i] = acc16[u][dt][i] * a2 + pv;
          }
        }
      }
    }

    if (n + 1 < nblk) lstore(buf ^ 1);
    __syncthreads();
  }

  // Epilogue: O / l -> FP16. Lane holds dims 32dt + 8g + 4hf + (0..3).
#pragma unroll
  for (int u = 0; u < SUB; ++u) {
    const float inv = 1.f / half_sum(lsum[u]);
    _Float16* orow = op + (size_t)(u * 32 + l32) * HD;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        h4 out;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float x;
          if constexpr (ACC16) x = (float)acc16[u][dt][(4 * g + e) >> 1][e & 1];
          else x = acc[u][dt][4 * g + e];
          out[e] = (_Float16)(x * inv);
        }
        *reinterpret_cast<h4*>(orow + dt * 32 + 8 * g + 4 * hf) = out;
      }
    }
  }
}

// Device entry points, one per accumulation variant. Their names contain the
// registry names of the backends that launch them, which is how the profiler
// attributes kernel time (WPE = waves per SIMD the register budget targets).
template <int NW, int SUB, int BN, int WPE>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
hip_fa_fp32acc_kernel(const _Float16* __restrict__ q, const _Float16* __restrict__ k,
                      const _Float16* __restrict__ vt, _Float16* __restrict__ o, int heads_q,
                      int group, int seq_q, int seq_k, float c) {
  fa_fwd_body<false, NW, SUB, BN>(q, k, vt, o, heads_q, group, seq_q, seq_k, c);
}

template <int NW, int SUB, int BN, int WPE>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
hip_fa_fp16acc_kernel(const _Float16* __restrict__ q, const _Float16* __restrict__ k,
                      const _Float16* __restrict__ vt, _Float16* __restrict__ o, int heads_q,
                      int group, int seq_q, int seq_k, float c) {
  fa_fwd_body<true, NW, SUB, BN>(q, k, vt, o, heads_q, group, seq_q, seq_k, c);
}

// ----------------------------------------------------------------------------
// Host side: tile table, validation, launch.

typedef void (*attn_fn)(const _Float16*, const _Float16*, const _Float16*, _Float16*, int, int,
                        int, int, float);

struct TileConfig {
  const char* name;
  int threads;
  int rows;        // BM
  int keys;        // BN
  attn_fn fp32;
  attn_fn fp16;
};

#define FA_TILE(NAME, NW, SUB, BN, WPE)                                                      \
  TileConfig {                                                                             \
    NAME, NW * 64, NW * SUB * 32, BN, &hip_fa_fp32acc_kernel<NW, SUB, BN, WPE>,            \
        &hip_fa_fp16acc_kernel<NW, SUB, BN, WPE>                                           \
  }

const TileConfig kTiles[] = {
    FA_TILE("w4_r64_n64", 4, 2, 64, 1),   // 4 waves x 64 rows, one wave per SIMD
    FA_TILE("w8_r32_n64", 8, 1, 64, 2),   // 8 waves x 32 rows, two waves per SIMD
};
constexpr int kNumTiles = sizeof(kTiles) / sizeof(kTiles[0]);
constexpr int kDefaultTile = 1;           // 1-based index into kTiles

int select_tile(const fa_problem* p, const TileConfig** out) {
  int idx = p->kernel == 0 ? kDefaultTile : p->kernel;
  if (idx < 1 || idx > kNumTiles) return FA_ERR_KERNEL;
  *out = &kTiles[idx - 1];
  return FA_OK;
}

int validate(const fa_problem* p, const TileConfig** tile) {
  if (!p) return FA_ERR_NULL;
  if (p->batch <= 0 || p->heads_q <= 0 || p->heads_kv <= 0 || p->seq_q <= 0 || p->seq_k <= 0 ||
      p->dim <= 0)
    return FA_ERR_GEOMETRY;
  if (p->heads_q % p->heads_kv) return FA_ERR_GEOMETRY;
  if (p->dim != HD) return FA_ERR_DIM;
  if (p->acc != FA_ACC_FP32 && p->acc != FA_ACC_FP16) return FA_ERR_ACC;
  if (!(p->scale > 0.f) || !isfinite(p->scale)) return FA_ERR_SCALE;
  if (p->reserved != 0) return FA_ERR_KERNEL;
  int rc = select_tile(p, tile);
  if (rc) return rc;
  // 32-bit index limits used inside the kernels.
  const int64_t lim = (int64_t)1 << 30;
  if (p->seq_q >= lim || p->seq_k >= lim || p->heads_q >= lim || p->batch >= lim)
    return FA_ERR_GEOMETRY;
  const int64_t bh = p->batch * p->heads_q;
  if (bh >= lim || (bh * (p->seq_q / (*tile)->rows)) >= lim || p->batch * p->heads_kv >= 65536)
    return FA_ERR_GEOMETRY;
  if (p->seq_q % (*tile)->rows || p->seq_k % (*tile)->keys || p->seq_k % VT_GROUP) return FA_ERR_TAIL;
  return FA_OK;
}

uint64_t workspace_for(const fa_problem* p) {
  return (uint64_t)p->batch * p->heads_kv * p->seq_k * p->dim * sizeof(_Float16);
}

}  // namespace

extern "C" {

int fa_fwd_workspace_bytes(const fa_problem* p, uint64_t* bytes) {
  if (!bytes) return FA_ERR_NULL;
  const TileConfig* tile = nullptr;
  int rc = validate(p, &tile);
  if (rc) return rc;
  *bytes = workspace_for(p);
  return FA_OK;
}

int fa_fwd_tile(const fa_problem* p, int32_t* rows, int32_t* keys) {
  if (!p || !rows || !keys) return FA_ERR_NULL;
  const TileConfig* tile = nullptr;
  int rc = select_tile(p, &tile);
  if (rc) return rc;
  *rows = tile->rows;
  *keys = tile->keys;
  return FA_OK;
}

int fa_fwd(const fa_problem* p, const void* q, const void* k, const void* v, void* o,
           void* workspace, uint64_t workspace_bytes, void* stream) {
  const TileConfig* tile = nullptr;
  int rc = validate(p, &tile);
  if (rc) return rc;
  if (!q || !k || !v || !o) return FA_ERR_NULL;
  if (!workspace || workspace_bytes < workspace_for(p)) return FA_ERR_WORKSPACE;
  for (const void* ptr : {q, k, v, (const void*)o, (const void*)workspace})
    if (reinterpret_cast<uintptr_t>(ptr) & 15) return FA_ERR_ALIGN;

  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int group = (int)(p->heads_q / p->heads_kv);
  _Float16* vt = static_cast<_Float16*>(workspace);

  (void)hipGetLastError();  // clear any stale error so the checks below see only ours
  dim3 vt_grid((unsigned)(p->seq_k / VT_GROUP), (unsigned)(p->batch * p->heads_kv));
  hipLaunchKernelGGL(fa_vt_kernel, vt_grid, dim3(256), 0, st, static_cast<const _Float16*>(v), vt,
                     (int)p->seq_k);
  if (hipGetLastError() != hipSuccess) return FA_ERR_LAUNCH;

  const double c = (double)p->scale * LOG2E;
  const unsigned grid = (unsigned)(p->batch * p->heads_q * (p->seq_q / tile->rows));
  attn_fn fn = p->acc == FA_ACC_FP16 ? tile->fp16 : tile->fp32;
  hipLaunchKernelGGL(fn, dim3(grid), dim3(tile->threads), 0, st, static_cast<const _Float16*>(q),
                     static_cast<const _Float16*>(k), static_cast<const _Float16*>(vt),
                     static_cast<_Float16*>(o), (int)p->heads_q, group, (int)p->seq_q,
                     (int)p->seq_k, (float)c);
  if (hipGetLastError() != hipSuccess) return FA_ERR_LAUNCH;
  return FA_OK;
}

int fa_kernel_count(void) { return kNumTiles; }

const char* fa_kernel_name(int32_t kernel) {
  if (kernel < 1 || kernel > kNumTiles) return nullptr;
  return kTiles[kernel - 1].name;
}

const char* fa_strerror(int status) {
  switch (status) {
    case FA_OK: return "ok";
    case FA_ERR_NULL: return "required pointer is NULL";
    case FA_ERR_GEOMETRY: return "invalid attention geometry";
    case FA_ERR_DIM: return "head dimension must be 128";
    case FA_ERR_TAIL: return "unsupported query/key tail: Nq or Nk not a multiple of the tile";
    case FA_ERR_ALIGN: return "tensor pointer not 16-byte aligned";
    case FA_ERR_WORKSPACE: return "workspace missing or too small";
    case FA_ERR_ACC: return "unknown accumulation variant";
    case FA_ERR_SCALE: return "scale must be finite and positive";
    case FA_ERR_KERNEL: return "unknown kernel selector";
    case FA_ERR_LAUNCH: return "HIP kernel launch failed";
    default: return "unknown status";
  }
}

}  // extern "C"
