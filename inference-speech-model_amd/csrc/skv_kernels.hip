// gfx950 kernels and C ABI for the decoder KV-cache hot path of a Whisper-class
// speech serving engine: paged append, block-table gather, paged decode
// attention and contiguous (cross-)attention. See speech_kv.h for the contract.
//
// Attention design (one launch, split-K with in-kernel merge):
//   * One wave64 owns one (query row, head, key chunk). A 16-byte lane load
//     carries EPL elements; LPT = D/EPL lanes cover one key row, so one wave
//     instruction reads TPI = 64/LPT whole key rows (128 contiguous bytes each
//     for fp16/bf16 at D=64) — fully coalesced per row.
//   * Each lane group (TPI groups per wave) keeps its own base-2 online-softmax
//     state over the keys it reads; the groups merge once at the end with lane
//     exchanges. K and V for U key rows per group are loaded before any math,
//     so a wave keeps U*2*16 B per lane (16 KB per wave at U=8) in flight.
//   * Waves of the same (row, head) write (m, l, acc) partials to scratch and
//     bump an arrival counter; the last arriving wave merges the partials,
//     writes the output and resets the counter to zero (so the counter buffer
//     needs zeroing once, and every launch is replay-safe inside a HIP graph).
#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "skv_device.h"
#include "speech_kv.h"

using namespace skv;

namespace {

thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail((int)e, "%s: launch failed: %s", what, hipGetErrorString(e));
  return SKV_OK;
}

int elt_bytes(int32_t dtype) {
  switch (dtype) {
    case SKV_F32: return 4;
    case SKV_F16: return 2;
    case SKV_BF16: return 2;
    default: return 0;
  }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------------------
// Append: pool[slot] = new row, 16 bytes per thread, K in grid.y 0, V in 1.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void append_kernel(const uint4* __restrict__ k_new, const uint4* __restrict__ v_new,
                                                     int64_t sn, int64_t sh, uint4* __restrict__ k_pool,
                                                     uint4* __restrict__ v_pool, const int64_t* __restrict__ slots,
                                                     int32_t n_tokens, int32_t heads, int32_t vpr, int64_t num_slots) {
  const uint4* src = blockIdx.y == 0 ? k_new : v_new;
  uint4* dst = blockIdx.y == 0 ? k_pool : v_pool;
  const int64_t per_tok = (int64_t)heads * vpr;
  const int64_t total = (int64_t)n_tokens * per_tok;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t n = i / per_tok;
    const int64_t r = i - n * per_tok;
    const int64_t h = r / vpr;
    const int64_t c = r - h * vpr;
    const int64_t slot = slots[n];
    if (slot < 0 || slot >= num_slots) continue;
    dst[slot * per_tok + r] = src[n * sn + h * sh + c];
  }
}

// ---------------------------------------------------------------------------
// Gather: out[b, h, t, :] = pool[table[b][t / bs] * bs + t % bs, h, :] for
// t < lens[b], zero otherwise. Output [B, H, T, D] contiguous.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void gather_kernel(const uint4* __restrict__ k_pool, const uint4* __restrict__ v_pool,
                                                     const int32_t* __restrict__ tables, int32_t tstride,
                                                     const int32_t* __restrict__ lens, uint4* __restrict__ k_out,
                                                     uint4* __restrict__ v_out, int32_t batch, int32_t heads, int32_t vpr,
                                                     int32_t bs, int32_t nb, int32_t T) {
  const uint4* src = blockIdx.y == 0 ? k_pool : v_pool;
  uint4* dst = blockIdx.y == 0 ? k_out : v_out;
  const int64_t per_head = (int64_t)T * vpr;
  const int64_t per_row = (int64_t)heads * per_head;
  const int64_t total = (int64_t)batch * per_row;
  const int64_t lim = (int64_t)tstride * bs;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = i / per_row;
    int64_t r = i - b * per_row;
    const int64_t h = r / per_head;
    r -= h * per_head;
    const int64_t t = r / vpr;
    const int64_t c = r - t * vpr;
    int64_t len = lens[b];
    len = len < T ? len : T;
    len = len < lim ? len : lim;
    uint4 val = make_uint4(0u, 0u, 0u, 0u);
    if (t < len) {
      const int32_t bi = (int32_t)(t / bs);
      const int32_t blk = tables[b * tstride + bi];
      if ((uint32_t)blk < (uint32_t)nb) {
        const int64_t tok = (int64_t)blk * bs + (t - (int64_t)bi * bs);
        val = src[(tok * heads + h) * vpr + c];
      }
    }
    dst[i] = val;
  }
}

// ---------------------------------------------------------------------------
// Attention.
// ---------------------------------------------------------------------------
struct AttnParams {
  const uint4* q;   // element strides below are in 16-byte vector units
  int64_t qsb, qsq, qsh;
  uint4* o;
  int64_t osb, osq, osh;
  const uint4* k;
  const uint4* v;
  // paged addressing
  const int32_t* tables;
  int32_t tstride;
  const int32_t* trows;
  int32_t bs, nb;
  int64_t row_vecs;  // vectors per pool token row = Hkv * D / EPL
  // contiguous addressing
  int64_t ss, sh, st;
  const int32_t* slots;
  // common
  const int32_t* lens;
  int32_t batch, qlen, heads, group, max_len, causal, chunk, nchunk_max;
  float scale_log2;
  float* part;      // [rows*heads*nchunk_max][D + 4]: m, l, -, -, acc[D]
  int32_t* counts;  // [rows*heads]
};

constexpr int kWavesPerBlock = 4;

template <int TPI>
constexpr int unroll_for() {
  return (64 / TPI) < 1 ? 1 : ((64 / TPI) > 8 ? 8 : (64 / TPI));
}

// Merge (m, l, acc) across the TPI lane groups of the wave (lane offsets
// LPT, 2*LPT, ..., 32).
template <int LPT, int EPL>
__device__ __forceinline__ void merge_groups(float& m, float& l, float* acc) {
#pragma unroll
  for (int off = LPT; off < 64; off <<= 1) {
    const float m2 = __shfl_xor(m, off, 64);
    const float l2 = __shfl_xor(l, off, 64);
    float a2[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) a2[e] = __shfl_xor(acc[e], off, 64);
    merge_state<EPL>(m, l, acc, m2, l2, a2);
  }
}

template <int DT, int D>
__device__ __forceinline__ void write_out(const AttnParams& p, int64_t o_off, float l, const float* acc) {
  constexpr int EPL = Elt<DT>::EPL;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  float r[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) r[e] = acc[e] * inv;
  p.o[o_off] = pack16<DT>(r);
}

template <int DT, int D, bool PAGED>
__global__ __launch_bounds__(256) void attention_kernel(AttnParams p) {
  constexpr int EPL = Elt<DT>::EPL;
  constexpr int LPT = D / EPL;
  constexpr int TPI = 64 / LPT;
  constexpr int U = unroll_for<TPI>();
  constexpr int PSTRIDE = D + 4;

  const int lane = threadIdx.x & 63;
  const int64_t wid = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  const int32_t rows = p.batch * p.qlen;
  const int64_t per_chunk = (int64_t)rows * p.heads;
  const int chunk = (int)(wid / per_chunk);
  if (chunk >= p.nchunk_max) return;
  const int64_t rh = wid - (int64_t)chunk * per_chunk;  // row * heads + head
  const int row = (int)(rh / p.heads);
  const int h = (int)(rh - (int64_t)row * p.heads);
  const int b = row / p.qlen;
  const int qi = row - b * p.qlen;

  int len = p.lens[b];
  if (p.causal) len -= (p.qlen - 1 - qi);
  len = len < 0 ? 0 : len;
  len = len > p.max_len ? p.max_len : len;
  const int g = lane / LPT;
  const int j = lane - g * LPT;
  const int64_t o_off = (int64_t)b * p.osb + (int64_t)qi * p.osq + (int64_t)h * p.osh + j;

  if (len == 0) {
    if (chunk == 0 && g == 0) p.o[o_off] = make_uint4(0u, 0u, 0u, 0u);
    return;
  }
  const int nchunks = (len + p.chunk - 1) / p.chunk;
  if (chunk >= nchunks) return;

  const uint4 qv = p.q[(int64_t)b * p.qsb + (int64_t)qi * p.qsq + (int64_t)h * p.qsh + j];
  const int kvh = h / p.group;

  const int32_t* tbl = nullptr;
  int64_t base = 0;
  if constexpr (PAGED) {
    const int trow = p.trows ? p.trows[b] : b;
    tbl = p.tables + (int64_t)trow * p.tstride;
    base = (int64_t)kvh * LPT + j;
  } else {
    const int slot = p.slots ? p.slots[b] : b;
    base = (int64_t)slot * p.ss + (int64_t)kvh * p.sh + j;
  }

  float m = kNegInf, l = 0.f;
  float acc[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) acc[e] = 0.f;

  const int t_begin = chunk * p.chunk;
  const int t_end = min(t_begin + p.chunk, len);
  for (int s = t_begin; s < t_end; s += TPI * U) {
    uint4 kr[U], vr[U];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = s + u * TPI + g;
      int64_t off = 0;
      bool valid = t < t_end;
      if constexpr (PAGED) {
        if (valid) {
          const int bi = t / p.bs;
          const int blk = tbl[bi];
          valid = (uint32_t)blk < (uint32_t)p.nb;
          off = ((int64_t)blk * p.bs + (t - bi * p.bs)) * p.row_vecs + base;
        }
      } else {
        off = base + (int64_t)t * p.st;
      }
      ok[u] = valid;
      if (valid) {
        kr[u] = load_stream(p.k + off);
        vr[u] = load_stream(p.v + off);
      } else {
        kr[u] = make_uint4(0u, 0u, 0u, 0u);
        vr[u] = make_uint4(0u, 0u, 0u, 0u);
      }
    }
    float sc[U];
    float mx = m;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float d = group_sum<LPT>(dot16<DT>(qv, kr[u]));
      sc[u] = ok[u] ? d * p.scale_log2 : kNegInf;
      mx = fmaxf(mx, sc[u]);
    }
    const float ref = (mx == kNegInf) ? 0.f : mx;
    const float alpha = __builtin_amdgcn_exp2f(m - ref);
    l *= alpha;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[e] *= alpha;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float pr = __builtin_amdgcn_exp2f(sc[u] - ref);
      l += pr;
      axpy16<DT>(pr, vr[u], acc);
    }
    m = mx;
  }

  merge_groups<LPT, EPL>(m, l, acc);

  if (nchunks == 1) {
    if (g == 0) write_out<DT, D>(p, o_off, l, acc);
    return;
  }

  // Split-K: publish this chunk's partial state, count arrivals.
  float* part = p.part + rh * (int64_t)p.nchunk_max * PSTRIDE;
  if (g == 0) {
    float4* dst = reinterpret_cast<float4*>(part + (int64_t)chunk * PSTRIDE + 4 + j * EPL);
#pragma unroll
    for (int e = 0; e < EPL; e += 4) dst[e / 4] = make_float4(acc[e], acc[e + 1], acc[e + 2], acc[e + 3]);
    if (j == 0) *reinterpret_cast<float2*>(part + (int64_t)chunk * PSTRIDE) = make_float2(m, l);
  }
  __threadfence();
  int ticket = 0;
  if (lane == 0) ticket = __hip_atomic_fetch_add(p.counts + rh, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
  ticket = __shfl(ticket, 0, 64);
  if (ticket != nchunks - 1) return;
  __threadfence();
  if (lane == 0) __hip_atomic_store(p.counts + rh, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // Last arrival: merge all chunk partials (lane group g takes chunks g, g+TPI, ...).
  float M = kNegInf, L = 0.f;
  float A[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) A[e] = 0.f;
  for (int c = g; c < nchunks; c += TPI) {
    const float* pc = part + (int64_t)c * PSTRIDE;
    const float2 ml = *reinterpret_cast<const float2*>(pc);
    float ac[EPL];
    const float4* src = reinterpret_cast<const float4*>(pc + 4 + j * EPL);
#pragma unroll
    for (int e = 0; e < EPL; e += 4) {
      const float4 x = src[e / 4];
      ac[e] = x.x;
      ac[e + 1] = x.y;
      ac[e + 2] = x.z;
      ac[e + 3] = x.w;
    }
    merge_state<EPL>(M, L, A, ml.x, ml.y, ac);
  }
  merge_groups<LPT, EPL>(M, L, A);
  if (g == 0) write_out<DT, D>(p, o_off, L, A);
}

// ---------------------------------------------------------------------------
// Host helpers.
// ---------------------------------------------------------------------------
constexpr int kPartPad = 4;

int64_t workspace_bytes(int64_t rows, int64_t heads, int64_t d, int64_t nchunk_max) {
  if (nchunk_max <= 1) return 0;
  return rows * heads * nchunk_max * (d + kPartPad) * (int64_t)sizeof(float);
}

int sub_tokens(int32_t dtype, int32_t d) {
  const int eb = elt_bytes(dtype);
  if (eb == 0 || d <= 0) return 0;
  const int epl = 16 / eb;
  const int lpt = d / epl;
  if (lpt <= 0) return 0;
  const int tpi = 64 / lpt;
  int u = 64 / tpi;
  u = u < 1 ? 1 : (u > 8 ? 8 : u);
  return tpi * u;
}

int32_t pick_chunk(int32_t rows, int32_t heads, int32_t d, int32_t max_len, int32_t dtype) {
  int sub = sub_tokens(dtype, d);
  if (sub <= 0) sub = 64;
  // Grow the chunk until the launch holds at most ~16K waves.
  const int64_t target = 16384;
  int64_t chunk = sub;
  while (chunk < max_len && (int64_t)rows * heads * cdiv(max_len, chunk) > target) chunk *= 2;
  return (int32_t)chunk;
}

bool supported_d(int32_t d) { return d == 16 || d == 32 || d == 64 || d == 128; }

template <int DT, int D, bool PAGED>
void launch_attention(const AttnParams& p, hipStream_t stream) {
  const int64_t waves = (int64_t)p.nchunk_max * p.batch * p.qlen * p.heads;
  const int64_t blocks = cdiv(waves, kWavesPerBlock);
  hipLaunchKernelGGL((attention_kernel<DT, D, PAGED>), dim3((uint32_t)blocks), dim3(64 * kWavesPerBlock), 0, stream, p);
}

template <bool PAGED>
int dispatch_attention(int32_t dtype, int32_t d, const AttnParams& p, hipStream_t stream) {
#define SKV_CASE(DT, DD)                          \
  if (dtype == DT && d == DD) {                   \
    launch_attention<DT, DD, PAGED>(p, stream);   \
    return SKV_OK;                                \
  }
  SKV_CASE(SKV_F16, 64) SKV_CASE(SKV_BF16, 64) SKV_CASE(SKV_F32, 64)
  SKV_CASE(SKV_F16, 16) SKV_CASE(SKV_BF16, 16) SKV_CASE(SKV_F32, 16)
  SKV_CASE(SKV_F16, 32) SKV_CASE(SKV_BF16, 32) SKV_CASE(SKV_F32, 32)
  SKV_CASE(SKV_F16, 128) SKV_CASE(SKV_BF16, 128) SKV_CASE(SKV_F32, 128)
#undef SKV_CASE
  return fail(SKV_EINVAL, "attention: unsupported dtype %d / head_dim %d", dtype, d);
}

// Shared validation + parameter fill for both attention entry points.
int prepare_attention(AttnParams& p, const char* who, const void* q, int64_t qsb, int64_t qsq, int64_t qsh,
                      const void* k, const void* v, void* out, int64_t osb, int64_t osq, int64_t osh,
                      const int32_t* lens, int32_t batch, int32_t q_len, int32_t heads, int32_t kv_heads,
                      int32_t d, int32_t max_len, float scale, int32_t causal, int32_t dtype, int32_t chunk,
                      void* ws, int64_t ws_bytes, int32_t* counters, int64_t counter_count) {
  const int eb = elt_bytes(dtype);
  if (eb == 0) return fail(SKV_EDTYPE, "%s: unknown dtype %d", who, dtype);
  if (!supported_d(d)) return fail(SKV_EINVAL, "%s: head_dim %d not in {16,32,64,128}", who, d);
  if (batch < 0 || q_len <= 0 || heads <= 0 || kv_heads <= 0 || heads % kv_heads != 0 || max_len < 0)
    return fail(SKV_EINVAL, "%s: bad sizes batch=%d q_len=%d heads=%d kv_heads=%d max_len=%d", who, batch, q_len,
                heads, kv_heads, max_len);
  if (!q || !k || !v || !out || !lens) return fail(SKV_EINVAL, "%s: null pointer argument", who);
  const int epl = 16 / eb;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
    return fail(SKV_EALIGN, "%s: q/k/v/out must be 16-byte aligned", who);
  if (qsb % epl || qsq % epl || qsh % epl || osb % epl || osq % epl || osh % epl)
    return fail(SKV_EALIGN, "%s: q/out strides must be multiples of %d elements", who, epl);
  if (chunk <= 0) chunk = pick_chunk(batch * q_len, heads, d, max_len, dtype);
  const int sub = sub_tokens(dtype, d);
  if (chunk % sub != 0) return fail(SKV_EINVAL, "%s: chunk_tokens %d must be a multiple of %d", who, chunk, sub);
  const int32_t nchunk_max = max_len > 0 ? (int32_t)cdiv(max_len, chunk) : 1;
  const int64_t need = workspace_bytes((int64_t)batch * q_len, heads, d, nchunk_max);
  if (need > 0 && (!ws || ws_bytes < need || !aligned16(ws)))
    return fail(SKV_EWORKSPACE, "%s: partials need %lld bytes (16-byte aligned), got %lld", who, (long long)need,
                (long long)ws_bytes);
  const int64_t need_cnt = (int64_t)batch * q_len * heads;
  if (need > 0 && (!counters || counter_count < need_cnt))
    return fail(SKV_EWORKSPACE, "%s: %lld zeroed int32 counters needed, got %lld", who, (long long)need_cnt,
                (long long)counter_count);
  p.q = (const uint4*)q;
  p.qsb = qsb / epl;
  p.qsq = qsq / epl;
  p.qsh = qsh / epl;
  p.o = (uint4*)out;
  p.osb = osb / epl;
  p.osq = osq / epl;
  p.osh = osh / epl;
  p.k = (const uint4*)k;
  p.v = (const uint4*)v;
  p.lens = lens;
  p.batch = batch;
  p.qlen = q_len;
  p.heads = heads;
  p.group = heads / kv_heads;
  p.max_len = max_len;
  p.causal = causal ? 1 : 0;
  p.chunk = chunk;
  p.nchunk_max = nchunk_max;
  p.scale_log2 = scale * kLog2e;
  p.part = need > 0 ? (float*)ws : nullptr;
  p.counts = need > 0 ? counters : nullptr;
  return SKV_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI.
// ---------------------------------------------------------------------------
extern "C" {

const char* skv_version(void) { return "speechkv 0.1.0 gfx950"; }

const char* skv_last_error(void) { return g_last_error; }

int skv_append(const void* k_new, const void* v_new, int64_t new_stride_n, int64_t new_stride_h, void* k_pool,
               void* v_pool, const int64_t* slot_mapping, int32_t n_tokens, int32_t num_heads, int32_t head_dim,
               int64_t num_slots, int32_t dtype, void* stream) {
  const int eb = elt_bytes(dtype);
  if (eb == 0) return fail(SKV_EDTYPE, "skv_append: unknown dtype %d", dtype);
  if (n_tokens < 0 || num_heads <= 0 || head_dim <= 0 || num_slots < 0)
    return fail(SKV_EINVAL, "skv_append: bad sizes n=%d heads=%d head_dim=%d slots=%lld", n_tokens, num_heads,
                head_dim, (long long)num_slots);
  if (n_tokens == 0) return SKV_OK;
  if (!k_new || !k_pool || !slot_mapping || ((v_new == nullptr) != (v_pool == nullptr)))
    return fail(SKV_EINVAL, "skv_append: null pointer argument");
  const int epl = 16 / eb;
  if (head_dim % epl) return fail(SKV_EALIGN, "skv_append: head_dim*%d bytes must be a multiple of 16", eb);
  if (!aligned16(k_new) || !aligned16(k_pool) || (v_new && (!aligned16(v_new) || !aligned16(v_pool))))
    return fail(SKV_EALIGN, "skv_append: pointers must be 16-byte aligned");
  if (new_stride_n % epl || new_stride_h % epl)
    return fail(SKV_EALIGN, "skv_append: strides must be multiples of %d elements", epl);
  const int vpr = head_dim / epl;
  const int64_t total = (int64_t)n_tokens * num_heads * vpr;
  int64_t blocks = cdiv(total, 256);
  if (blocks > 65535) blocks = 65535;
  hipLaunchKernelGGL(append_kernel, dim3((uint32_t)blocks, v_new ? 2 : 1), dim3(256), 0, (hipStream_t)stream,
                     (const uint4*)k_new, (const uint4*)(v_new ? v_new : k_new), new_stride_n / epl,
                     new_stride_h / epl, (uint4*)k_pool, (uint4*)(v_pool ? v_pool : k_pool), slot_mapping, n_tokens,
                     num_heads, vpr, num_slots);
  return check_launch("skv_append");
}

int skv_gather(const void* k_pool, const void* v_pool, const int32_t* block_tables, int32_t table_stride,
               const int32_t* lens, void* k_out, void* v_out, int32_t batch, int32_t num_heads, int32_t head_dim,
               int32_t block_size, int32_t num_blocks, int32_t max_len, int32_t dtype, void* stream) {
  const int eb = elt_bytes(dtype);
  if (eb == 0) return fail(SKV_EDTYPE, "skv_gather: unknown dtype %d", dtype);
  if (batch < 0 || num_heads <= 0 || head_dim <= 0 || block_size <= 0 || num_blocks < 0 || max_len < 0 ||
      table_stride < 0)
    return fail(SKV_EINVAL, "skv_gather: bad sizes");
  if (batch == 0 || max_len == 0) return SKV_OK;
  if (!k_pool || !k_out || !block_tables || !lens || ((v_pool == nullptr) != (v_out == nullptr)))
    return fail(SKV_EINVAL, "skv_gather: null pointer argument");
  const int epl = 16 / eb;
  if (head_dim % epl) return fail(SKV_EALIGN, "skv_gather: head_dim*%d bytes must be a multiple of 16", eb);
  if (!aligned16(k_pool) || !aligned16(k_out) || (v_pool && (!aligned16(v_pool) || !aligned16(v_out))))
    return fail(SKV_EALIGN, "skv_gather: pointers must be 16-byte aligned");
  const int vpr = head_dim / epl;
  const int64_t total = (int64_t)batch * num_heads * max_len * vpr;
  int64_t blocks = cdiv(total, 256);
  if (blocks > 65535) blocks = 65535;
  hipLaunchKernelGGL(gather_kernel, dim3((uint32_t)blocks, v_pool ? 2 : 1), dim3(256), 0, (hipStream_t)stream,
                     (const uint4*)k_pool, (const uint4*)(v_pool ? v_pool : k_pool), block_tables, table_stride, lens,
                     (uint4*)k_out, (uint4*)(v_out ? v_out : k_out), batch, num_heads, vpr, block_size, num_blocks,
                     max_len);
  return check_launch("skv_gather");
}

int64_t skv_attention_workspace_bytes(int32_t rows, int32_t num_heads, int32_t head_dim, int32_t max_len,
                                      int32_t chunk_tokens, int32_t dtype) {
  if (rows <= 0 || num_heads <= 0 || head_dim <= 0 || max_len <= 0 || elt_bytes(dtype) == 0) return 0;
  if (chunk_tokens <= 0) chunk_tokens = pick_chunk(rows, num_heads, head_dim, max_len, dtype);
  return workspace_bytes(rows, num_heads, head_dim, cdiv(max_len, chunk_tokens));
}

int32_t skv_default_chunk_tokens(int32_t rows, int32_t num_heads, int32_t head_dim, int32_t max_len, int32_t dtype) {
  return pick_chunk(rows, num_heads, head_dim, max_len, dtype);
}

int skv_paged_attention(const void* q, int64_t q_stride_b, int64_t q_stride_q, int64_t q_stride_h,
                        const void* k_pool, const void* v_pool, const int32_t* block_tables, int32_t table_stride,
                        const int32_t* table_rows, const int32_t* ctx_lens, void* out, int64_t o_stride_b,
                        int64_t o_stride_q, int64_t o_stride_h, int32_t batch, int32_t q_len, int32_t num_heads,
                        int32_t num_kv_heads, int32_t head_dim, int32_t block_size, int32_t num_blocks,
                        int32_t max_ctx, float scale, int32_t causal, int32_t dtype, int32_t chunk_tokens,
                        void* partials, int64_t partial_bytes, int32_t* counters, int64_t counter_count,
                        void* stream) {
  if (block_size <= 0 || num_blocks < 0 || table_stride <= 0 || !block_tables)
    return fail(SKV_EINVAL, "skv_paged_attention: bad block table arguments");
  const int64_t table_cap = (int64_t)table_stride * block_size;
  if (max_ctx > table_cap) max_ctx = (int32_t)table_cap;
  AttnParams p{};
  int rc = prepare_attention(p, "skv_paged_attention", q, q_stride_b, q_stride_q, q_stride_h, k_pool, v_pool, out,
                             o_stride_b, o_stride_q, o_stride_h, ctx_lens, batch, q_len, num_heads, num_kv_heads,
                             head_dim, max_ctx, scale, causal, dtype, chunk_tokens, partials, partial_bytes,
                             counters, counter_count);
  if (rc != SKV_OK) return rc;
  if (batch == 0) return SKV_OK;
  p.tables = block_tables;
  p.tstride = table_stride;
  p.trows = table_rows;
  p.bs = block_size;
  p.nb = num_blocks;
  p.row_vecs = (int64_t)num_kv_heads * head_dim / (16 / elt_bytes(dtype));
  rc = dispatch_attention<true>(dtype, head_dim, p, (hipStream_t)stream);
  if (rc != SKV_OK) return rc;
  return check_launch("skv_paged_attention");
}

int skv_dense_attention(const void* q, int64_t q_stride_b, int64_t q_stride_q, int64_t q_stride_h, const void* k,
                        const void* v, int64_t kv_stride_s, int64_t kv_stride_h, int64_t kv_stride_t,
                        const int32_t* slot_ids, const int32_t* lens, void* out, int64_t o_stride_b,
                        int64_t o_stride_q, int64_t o_stride_h, int32_t batch, int32_t q_len, int32_t num_heads,
                        int32_t num_kv_heads, int32_t head_dim, int32_t max_len, float scale, int32_t causal,
                        int32_t dtype, int32_t chunk_tokens, void* partials, int64_t partial_bytes,
                        int32_t* counters, int64_t counter_count, void* stream) {
  AttnParams p{};
  int rc = prepare_attention(p, "skv_dense_attention", q, q_stride_b, q_stride_q, q_stride_h, k, v, out, o_stride_b,
                             o_stride_q, o_stride_h, lens, batch, q_len, num_heads, num_kv_heads, head_dim, max_len,
                             scale, causal, dtype, chunk_tokens, partials, partial_bytes, counters, counter_count);
  if (rc != SKV_OK) return rc;
  const int epl = 16 / elt_bytes(dtype);
  if (kv_stride_s % epl || kv_stride_h % epl || kv_stride_t % epl)
    return fail(SKV_EALIGN, "skv_dense_attention: K/V strides must be multiples of %d elements", epl);
  if (batch == 0) return SKV_OK;
  p.ss = kv_stride_s / epl;
  p.sh = kv_stride_h / epl;
  p.st = kv_stride_t / epl;
  p.slots = slot_ids;
  rc = dispatch_attention<false>(dtype, head_dim, p, (hipStream_t)stream);
  if (rc != SKV_OK) return rc;
  return check_launch("skv_dense_attention");
}

}  // extern "C"
