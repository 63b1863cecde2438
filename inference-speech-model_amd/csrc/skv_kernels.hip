// gfx950 kernels and C ABI for the decoder KV-cache hot path of a Whisper-class
// speech serving engine: paged append, block-table gather, paged decode
// attention and contiguous (cross-)attention. See speech_kv.h for the contract.
//
// Attention design:
//   * One workgroup of kWaves wave64s owns one (query row, head, key chunk).
//     Paged fast path (power-of-two block size of at least TPI keys): each
//     wave reads its block ids with scalar loads, one batch per trip, and no
//     load the wave issues before its first K/V loads is waited for: a CU
//     returns vector loads in issue order, so a vector table (or q) load of a
//     workgroup that starts late would wait behind the K/V bytes already
//     queued by the CU's other workgroups. General paged path: the chunk's
//     block ids are staged once into LDS.
//   * A 16-byte lane load carries EPL elements; LPT = D/EPL lanes cover one
//     key row, so one wave instruction reads TPI = 64/LPT whole key rows
//     (128 contiguous bytes each for fp16/bf16 at D=64). A wave loads K and V
//     for U rows per lane group (a SUB = TPI*U-key sub-chunk) before any math.
//   * Each lane group keeps its own base-2 online-softmax state; groups merge
//     with lane exchanges, then the kWaves waves merge through LDS.
//   * A row whose keys span several chunks writes one (m, l, acc) partial per
//     chunk; merge_kernel (same stream, next launch) combines them. The kernel
//     boundary orders the two, so no device-scope fence runs inside a kernel.
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>
#include <type_traits>

#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "skv_common.h"
#include "skv_device.h"
#include "speech_kv.h"

namespace skv {

namespace {
thread_local char g_last_error[512] = "";
}  // namespace

const char* last_error() { return g_last_error; }

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

}  // namespace skv

using namespace skv;

namespace {

// ---------------------------------------------------------------------------
// Append: pool[slot] = new row, 16 bytes per thread, K in grid.y 0, V in 1.
// Loads and stores carry the nontemporal hint: at the encoder-store size (64 x 1500
// rows of 20 x 64 bf16 per K and V) that is 2.5% faster than the default policy.
// ---------------------------------------------------------------------------
// Division by a launch-constant divisor d without a divide: m = floor(2^32 / d)
// (2^32 - 1 for d = 1), so umulhi(n, m) is floor(n / d) or one less for every
// n < 2^32, and one remainder test corrects it.
struct DivU32 {
  uint32_t d, m;
};
DivU32 make_div(uint32_t d) { return {d, d == 1 ? 0xffffffffu : (uint32_t)((1ull << 32) / d)}; }
__device__ __forceinline__ uint32_t udiv(uint32_t n, DivU32 f) {
  uint32_t q = __umulhi(n, f.m);
  if (n - q * f.d >= f.d) ++q;
  return q;
}

// Append with 32-bit element indices (total rows * heads * vectors < 2^31).
__global__ __launch_bounds__(256) void append32_kernel(const uint4* __restrict__ k_new, const uint4* __restrict__ v_new,
                                                       int64_t sn, int64_t sh, uint4* __restrict__ k_pool,
                                                       uint4* __restrict__ v_pool, const int64_t* __restrict__ slots,
                                                       uint32_t total, DivU32 per_tok, DivU32 vpr, int64_t num_slots) {
  const uint4* src = blockIdx.y == 0 ? k_new : v_new;
  uint4* dst = blockIdx.y == 0 ? k_pool : v_pool;
  for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < total; i += gridDim.x * 256u) {
    const uint32_t n = udiv(i, per_tok);
    const uint32_t r = i - n * per_tok.d;
    const uint32_t h = udiv(r, vpr);
    const uint32_t c = r - h * vpr.d;
    const int64_t slot = slots[n];
    if (slot < 0 || slot >= num_slots) continue;
    store_stream(dst + slot * per_tok.d + r, load_stream(src + (int64_t)n * sn + (int64_t)h * sh + c));
  }
}

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
    store_stream(dst + slot * per_tok + r, load_stream(src + n * sn + h * sh + c));
  }
}

// ---------------------------------------------------------------------------
// Gather: out[b, h, t, :] = pool[table[b][t / bs] * bs + t % bs, h, :] for
// t < lens[b], zero otherwise. Output [B, H, T, D] contiguous.
// ---------------------------------------------------------------------------
// Gather with 32-bit element indices (total output vectors < 2^31). One thread
// copies one 16-byte column c of kGatherRows consecutive token rows of one
// (row, head): one length read, then the rows' table reads and their pool
// loads, all independent of each other, so each thread has kGatherRows loads
// in flight. Output rows past the length (up to T) are written as zeros.
// Pool rows are read with the nontemporal hint; the output keeps the default store
// policy (nontemporal stores were 10% slower at the large-v3 decode batch).
constexpr int kGatherRows = 4;
__global__ __launch_bounds__(256) void gather32_kernel(const uint4* __restrict__ k_pool, const uint4* __restrict__ v_pool,
                                                       const int32_t* __restrict__ tables, int32_t tstride,
                                                       const int32_t* __restrict__ lens, uint4* __restrict__ k_out,
                                                       uint4* __restrict__ v_out, uint32_t total, DivU32 per_row,
                                                       DivU32 per_head, DivU32 vpr, DivU32 bs, int32_t heads, int32_t nb,
                                                       int32_t T) {
  const uint4* src = blockIdx.y == 0 ? k_pool : v_pool;
  uint4* dst = blockIdx.y == 0 ? k_out : v_out;
  const int64_t lim = (int64_t)tstride * bs.d;
  for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < total; i += gridDim.x * 256u) {
    // i enumerates (b, h, row group, c) with per_head = ceil(T / kGatherRows) * vpr.
    const uint32_t b = udiv(i, per_row);
    uint32_t r = i - b * per_row.d;
    const uint32_t h = udiv(r, per_head);
    r -= h * per_head.d;
    const uint32_t tg = udiv(r, vpr);
    const uint32_t c = r - tg * vpr.d;
    const uint32_t t0 = tg * kGatherRows;
    int64_t len = lens[b];
    len = len < T ? len : T;
    len = len < lim ? len : lim;
    uint4 val[kGatherRows];
#pragma unroll
    for (int u = 0; u < kGatherRows; ++u) {
      const uint32_t t = t0 + u;
      val[u] = make_uint4(0u, 0u, 0u, 0u);
      if ((int64_t)t < len) {
        const uint32_t bi = udiv(t, bs);
        const int32_t blk = tables[(int64_t)b * tstride + bi];
        if ((uint32_t)blk < (uint32_t)nb) {
          const int64_t tok = (int64_t)blk * bs.d + (t - bi * bs.d);
          val[u] = load_stream(src + (tok * heads + h) * vpr.d + c);
        }
      }
    }
    const uint32_t o = ((b * (uint32_t)heads + h) * (uint32_t)T + t0) * vpr.d + c;
#pragma unroll
    for (int u = 0; u < kGatherRows; ++u)
      if (t0 + u < (uint32_t)T) dst[o + u * vpr.d] = val[u];
  }
}

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
        val = load_stream(src + (tok * heads + h) * vpr + c);
      }
    }
    dst[i] = val;
  }
}

// Gather by waves (a power-of-two block size of at least 64 / vpr keys, a pool of at
// most 2 GiB): one wave copies kGatherLoads * 64 / vpr consecutive token rows of one
// (row, head), 64 / vpr rows per load instruction (vpr lanes per row). The rows of
// one instruction lie in one block, so its block id is wave-uniform: the row length
// and the instructions' block ids (their table index clamped to the row) load in one
// scalar batch, and the pool loads follow after that single round trip. Pool rows
// are read with buffer loads against a descriptor of the pool; a row at or past the
// length, or behind a block id outside the pool, gets an out-of-range offset, for
// which the hardware returns zeros without a memory access, so the padding costs no
// read and no load is predicated. Output rows past T (the last group) are not stored.
// The arguments of the address chain come first, as plain scalars (the divisors'
// fields apart: preloading stops at an aggregate): the build preloads the first
// argument dwords into scalar registers, so the chain starts without an argument load.
constexpr int kGatherLoads = 4;
__global__ __launch_bounds__(256) void gather_rows_kernel(uint32_t waves, uint32_t row_d, uint32_t row_m,
                                                          uint32_t head_d, uint32_t head_m, int32_t tstride,
                                                          int32_t bs_shift, int32_t vpr_shift,
                                                          const int32_t* __restrict__ tables,
                                                          const int32_t* __restrict__ lens, int32_t T, int32_t nb,
                                                          int32_t heads, uint32_t pool_bytes,
                                                          const uint4* __restrict__ k_pool,
                                                          const uint4* __restrict__ v_pool, uint4* __restrict__ k_out,
                                                          uint4* __restrict__ v_out) {
  const uint32_t w = blockIdx.x * 4u + (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  if (w >= waves) return;
  const DivU32 per_row{row_d, row_m}, per_head{head_d, head_m};
  const uint4* src = blockIdx.y == 0 ? k_pool : v_pool;
  uint4* dst = blockIdx.y == 0 ? k_out : v_out;
  const int lane = threadIdx.x & 63;
  const uint32_t b = udiv(w, per_row);
  const uint32_t r = w - b * per_row.d;
  const uint32_t h = udiv(r, per_head);
  const uint32_t grp = r - h * per_head.d;
  const int rpi = 64 >> vpr_shift;  // rows per load instruction
  const int t0 = (int)grp * rpi * kGatherLoads;
  const int32_t* trow = tables + (int64_t)b * tstride;
  int len = lens[b];
  uint32_t blk[kGatherLoads];
#pragma unroll
  for (int u = 0; u < kGatherLoads; ++u) blk[u] = (uint32_t)trow[min((t0 + u * rpi) >> bs_shift, tstride - 1)];
  asm volatile("" ::"s"(len), "s"(blk[0]), "s"(blk[1]), "s"(blk[2]), "s"(blk[3]));
  const int64_t lim = (int64_t)tstride << bs_shift;
  len = len < 0 ? 0 : (len > T ? T : len);
  len = (int64_t)len < lim ? len : (int)lim;
  const uint32_t row_bytes = ((uint32_t)heads << vpr_shift) * 16u;  // one token row of every head
  const int row = lane >> vpr_shift;
  const uint32_t col = ((h << vpr_shift) + (uint32_t)(lane & ((1 << vpr_shift) - 1))) * 16u;
  const __amdgpu_buffer_rsrc_t res =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint4*>(src), (short)0, (int)pool_bytes, kBufWord3);
  const uint32_t bmask = (1u << bs_shift) - 1u;
  uint4 val[kGatherLoads];
#pragma unroll
  for (int u = 0; u < kGatherLoads; ++u) {
    const int t = t0 + u * rpi + row;
    const uint32_t off = t < len && blk[u] < (uint32_t)nb
                             ? ((blk[u] << bs_shift) + ((uint32_t)t & bmask)) * row_bytes + col
                             : kBufOutOfRange;
    const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(res, off, 0, kBufNt);
    val[u] = make_uint4(x.x, x.y, x.z, x.w);
  }
  const uint32_t o = ((b * (uint32_t)heads + h) * (uint32_t)T + (uint32_t)t0 + (uint32_t)row) << vpr_shift |
                     (uint32_t)(lane & ((1 << vpr_shift) - 1));
#pragma unroll
  for (int u = 0; u < kGatherLoads; ++u)
    if (t0 + u * rpi + row < T) dst[o + ((uint32_t)(u * rpi) << vpr_shift)] = val[u];
}

// ---------------------------------------------------------------------------
// Encoder K/V into a decode slot: for every (layer, K|V) source and head h the
// first n positions (rows of D elements) are copied into the slot's region of
// the slot-major cross-attention buffer. Grid: z = layer * 2 + kv, y = head, x
// covers the head's n * vpr 16-byte vectors, kCopyVecs per thread (all loads
// issued before the stores). Nontemporal loads and stores: 11% faster than the
// default policy for a request's 32 layers of 1500 x 20 x 64 bf16.
// ---------------------------------------------------------------------------
constexpr int kMaxCrossLayers = 64;
constexpr int kCopyVecs = 4;

struct CrossCopyParams {
  const uint4* src[2 * kMaxCrossLayers];  // layer l: K at 2l, V at 2l + 1
  int64_t ssh, sst;                       // source head / position strides, 16-byte vectors
  uint4* dst;
  int64_t dsl, dskv, dsh, dst_t;          // destination layer / kv / head / position strides
  int32_t n, vpr, vpr_shift;              // positions, vectors per row, log2(vpr) (vpr is 2^k)
};

__global__ __launch_bounds__(256) void cross_copy_kernel(CrossCopyParams p) {
  const int pair = blockIdx.z;
  const int h = blockIdx.y;
  const uint4* src = p.src[pair] + (int64_t)h * p.ssh;
  uint4* dst = p.dst + (int64_t)(pair >> 1) * p.dsl + (int64_t)(pair & 1) * p.dskv + (int64_t)h * p.dsh;
  const int64_t total = (int64_t)p.n * p.vpr;
  const int64_t step = (int64_t)gridDim.x * 256;
  for (int64_t i0 = (int64_t)blockIdx.x * 256 + threadIdx.x; i0 < total; i0 += step * kCopyVecs) {
    uint4 v[kCopyVecs];
#pragma unroll
    for (int u = 0; u < kCopyVecs; ++u) {
      const int64_t i = i0 + u * step;
      if (i < total) {
        const int64_t t = i >> p.vpr_shift;
        v[u] = load_stream(src + t * p.sst + (i & (p.vpr - 1)));
      }
    }
#pragma unroll
    for (int u = 0; u < kCopyVecs; ++u) {
      const int64_t i = i0 + u * step;
      if (i < total) {
        const int64_t t = i >> p.vpr_shift;
        store_stream(dst + t * p.dst_t + (i & (p.vpr - 1)), v[u]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Greedy sampling: out[r] = first index of the maximum of logits[r, :vocab]
// (NaN counts as the maximum, as in torch.argmax). Optionally, for a row whose
// slot s = row_slots[r] is in [0, num_slots): slot_tokens[s] = token (the next
// step's input), and when the token is the slot's EOS id (slot_eos[s] >= 0) and
// the slot is not yet finished, slot_finished[s] = 1 and finished_count += 1.
// One workgroup per row reads the row as 16-byte vectors of 32-bit words through a
// buffer descriptor (reads past the row's last word return zeros and are not
// compared), VECS vectors per thread in flight. A thread visits its elements
// in increasing index order and keeps the first strictly greater value: per element a
// compare and two selects (the value, and the element's position in the pass, a
// constant; the position becomes an index once per pass). A NaN-propagating running
// maximum (one instruction per two elements) flags a NaN, and a thread that saw one
// rescans its elements for the first NaN (NaN counts as the maximum). A 16-bit row
// that starts in the middle of a word has its first element handled alone. The
// threads' (value, index) candidates are reduced over each wave's lanes with DPP and
// permlane exchanges (no LDS round trip per step), then over the waves through LDS.
// ---------------------------------------------------------------------------
constexpr int kArgmaxThreads = 1024;
// 16-byte vectors per thread per pass (VECS): the launch takes the fewest of 1, 2, 4, 7 that
// cover a row in one pass (7: up to 57344 16-bit logits, so the 51866-entry Whisper vocabulary
// is one pass); larger rows take several passes of 7.

__device__ __forceinline__ bool argmax_better(float v1, int i1, float v2, int i2) {
  const bool n1 = v1 != v1, n2 = v2 != v2;
  if (n1 || n2) return n1 && (!n2 || i1 < i2);
  return v1 > v2 || (v1 == v2 && i1 < i2);
}

template <int DT> __device__ __forceinline__ float half_word(uint32_t w, int hi);
template <> __device__ __forceinline__ float half_word<SKV_F16>(uint32_t w, int hi) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(hi ? w >> 16 : w & 0xffffu));
}
template <> __device__ __forceinline__ float half_word<SKV_BF16>(uint32_t w, int hi) {
  return __uint_as_float(hi ? (w & 0xffff0000u) : (w << 16));
}
template <int DT> __device__ __forceinline__ float word_elt(uint32_t w, int e) {
  if constexpr (DT == SKV_F32) {
    return __uint_as_float(w);
  } else {
    return half_word<DT>(w, e);
  }
}

struct SlotFeedback {
  const int32_t* row_slots;  // NULL: no per-slot output
  int32_t num_slots;
  int64_t* slot_tokens;      // optional
  const int64_t* slot_eos;   // optional, with slot_finished and finished_count
  int32_t* slot_finished;
  unsigned long long* finished_count;
};

template <int DT, int VECS>
__global__ __launch_bounds__(kArgmaxThreads) void argmax_kernel(const char* __restrict__ logits, int64_t row_bytes,
                                                                int32_t vocab, int64_t* __restrict__ out,
                                                                SlotFeedback f) {
  constexpr int kAmWaves = kArgmaxThreads / 64;
  __shared__ float s_v[kAmWaves];
  __shared__ int s_i[kAmWaves];
  const int r = blockIdx.x;
  const char* row = logits + (int64_t)r * row_bytes;
  // Elements per word, the element held alone before the first word, and the word count.
  constexpr int EPW = DT == SKV_F32 ? 1 : 2;
  const int head = (EPW == 2 && ((uintptr_t)row & 3u)) ? 1 : 0;
  const char* words = row + head * 2;
  const int nw = (vocab - head) / EPW;
  const __amdgpu_buffer_rsrc_t res =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(words), (short)0, nw * 4, kBufWord3);
  // The candidate starts at the thread's first element (value -inf), so a row whose maximum is
  // -inf resolves to its first index like the others.
  float best = kNegInf;
  int bi = 4 * (int)threadIdx.x < nw ? head + EPW * 4 * (int)threadIdx.x : 0x7fffffff;
  float nmax = kNegInf;  // NaN-propagating maximum of the thread's elements: NaN flags a NaN
  // Slot feedback inputs load while the row streams in: wave 0, which writes the feedback, reads
  // the row's slot and then the slot's EOS id and finished flag once its first pass's loads are
  // issued, so the end of the kernel waits for no dependent load. Empty asm statements with a
  // memory clobber keep these loads behind the pass's loads.
  const bool wave0 = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)) == 0;
  int slot = -1;
  int64_t slot_eos = -1;
  int slot_fin = 1;
  // Thread t's vectors: words 4 * (t + kArgmaxThreads * k) .. +3, k = 0, 1, ...
  constexpr int kPassWords = 4 * kArgmaxThreads * VECS;
  constexpr int kVecElts = 4 * EPW;
  for (int p0 = 0; p0 < nw; p0 += kPassWords) {
    u32x4 x[VECS];
#pragma unroll
    for (int k = 0; k < VECS; ++k)
      x[k] = __builtin_amdgcn_raw_buffer_load_b128(
          res, (uint32_t)(p0 + 4 * ((int)threadIdx.x + kArgmaxThreads * k)) * 4u, 0, kBufNt);
    if (p0 == 0 && wave0 && f.row_slots) {
      slot = f.row_slots[r];
      if (slot >= 0 && slot < f.num_slots && f.slot_eos) {
        slot_eos = f.slot_eos[slot];
        slot_fin = f.slot_finished[slot];
      }
    }
    // The pass's winner is kept as its position k * kVecElts + (EPW * j + e), a constant of
    // the unrolled loop (-1: none), and turned into an element index once per pass.
    int pos = -1;
    auto visit = [&](float v, int at) __attribute__((always_inline)) {
      const bool gt = v > best;
      best = gt ? v : best;
      pos = gt ? at : pos;
    };
#pragma unroll
    for (int k = 0; k < VECS; ++k) {
      const int w0 = p0 + 4 * ((int)threadIdx.x + kArgmaxThreads * k);
      if (w0 + 4 <= nw) {  // a whole vector inside the row
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float v[EPW];
#pragma unroll
          for (int e = 0; e < EPW; ++e) v[e] = word_elt<DT>(x[k][j], e);
          if constexpr (EPW == 2)
            nmax = max_score(nmax, max_score(v[0], v[1]));
          else
            nmax = max_score(nmax, v[0]);
#pragma unroll
          for (int e = 0; e < EPW; ++e) visit(v[e], k * kVecElts + EPW * j + e);
        }
      } else if (w0 < nw) {  // the row's last vector, partly past its end
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int e = 0; e < EPW; ++e) {
            const float v = j < nw - w0 ? word_elt<DT>(x[k][j], e) : kNegInf;
            nmax = max_score(nmax, v);
            visit(v, k * kVecElts + EPW * j + e);
          }
      }
    }
    if (pos >= 0) {
      const int k = pos / kVecElts;
      bi = head + EPW * (p0 + 4 * ((int)threadIdx.x + kArgmaxThreads * k)) + (pos - k * kVecElts);
    }
  }
  const bool nan_seen = nmax != nmax;
  if (nan_seen) {  // rare: the first NaN among this thread's elements wins
    int ni = 0x7fffffff;
    for (int p0 = 0; p0 < nw; p0 += kPassWords)
      for (int k = 0; k < VECS; ++k) {
        const int w0 = p0 + 4 * ((int)threadIdx.x + kArgmaxThreads * k);
        const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(res, (uint32_t)w0 * 4u, 0, kBufNt);
        for (int j = 0; j < 4; ++j)
          for (int e = 0; e < EPW; ++e) {
            const float v = word_elt<DT>(x[j], e);
            const int i = head + EPW * (w0 + j) + e;
            if (w0 + j < nw && v != v && i < ni) ni = i;
          }
      }
    if (ni != 0x7fffffff) {
      best = __builtin_nanf("");
      bi = ni;
    }
  }
  auto consider = [&](float v, int i) {
    if (argmax_better(v, i, best, bi)) {
      best = v;
      bi = i;
    }
  };
  if constexpr (EPW == 2) {
    if (threadIdx.x == 0) {
      const uint16_t* e = reinterpret_cast<const uint16_t*>(row);
      if (head) consider(half_word<DT>(e[0], 0), 0);
      if ((vocab - head) & 1) consider(half_word<DT>(e[vocab - 1], 0), vocab - 1);
    }
  }
  // (value, index) pairs reduced over lanes with DPP and permlane exchanges (every lane active).
  auto step = [&](auto off_c) __attribute__((always_inline)) {
    constexpr int OFF = decltype(off_c)::value;
    consider(xor_lane<OFF>(best), __float_as_int(xor_lane<OFF>(__int_as_float(bi))));
  };
  step(std::integral_constant<int, 32>{});
  step(std::integral_constant<int, 16>{});
  step(std::integral_constant<int, 8>{});
  step(std::integral_constant<int, 4>{});
  step(std::integral_constant<int, 2>{});
  step(std::integral_constant<int, 1>{});
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    s_v[wave] = best;
    s_i[wave] = bi;
  }
  __syncthreads();
  if (wave != 0) return;
  const int lane = threadIdx.x;
  best = lane < kAmWaves ? s_v[lane] : kNegInf;
  bi = lane < kAmWaves ? s_i[lane] : 0x7fffffff;
  static_assert(kAmWaves == 16, "the final reduction covers 16 waves");
  step(std::integral_constant<int, 8>{});
  step(std::integral_constant<int, 4>{});
  step(std::integral_constant<int, 2>{});
  step(std::integral_constant<int, 1>{});
  if (lane == 0) {
    const int64_t tok = bi == 0x7fffffff ? 0 : bi;
    out[r] = tok;
    if (slot >= 0 && slot < f.num_slots) {
      if (f.slot_tokens) f.slot_tokens[slot] = tok;
      // Rows name distinct slots within one launch (idle rows name a slot with no EOS), so the
      // finished flag has one writer (read above, before this row's store); the count is shared.
      if (slot_eos >= 0 && tok == slot_eos && slot_fin == 0) {
        f.slot_finished[slot] = 1;
        atomicAdd(f.finished_count, 1ull);
      }
    }
  }
}

template <int DT>
void launch_argmax(int vecs, int32_t rows, hipStream_t s, const char* logits, int64_t rb, int32_t vocab, int64_t* out,
                   const SlotFeedback& f) {
  const dim3 grid((uint32_t)rows), block(kArgmaxThreads);
  switch (vecs) {
    case 1: hipLaunchKernelGGL((argmax_kernel<DT, 1>), grid, block, 0, s, logits, rb, vocab, out, f); break;
    case 2: hipLaunchKernelGGL((argmax_kernel<DT, 2>), grid, block, 0, s, logits, rb, vocab, out, f); break;
    case 4: hipLaunchKernelGGL((argmax_kernel<DT, 4>), grid, block, 0, s, logits, rb, vocab, out, f); break;
    default: hipLaunchKernelGGL((argmax_kernel<DT, 7>), grid, block, 0, s, logits, rb, vocab, out, f); break;
  }
}

// ---------------------------------------------------------------------------
// Residual add + LayerNorm of a decode batch (the pre-LN transformer's
// `x = x + f(x); h = norm(x)`): sum = x + y rounded to the tensor type, as the
// separate add would store it; norm = (sum - mean) / sqrt(var + eps) * gamma +
// beta over the row with fp32 statistics (population variance, two passes over
// registers), as torch.nn.LayerNorm computes it. One wave per row holds the row
// in registers: VPL 16-byte vectors per lane.
// ---------------------------------------------------------------------------
template <int DT> __device__ __forceinline__ void unpack16(const uint4& v, float* f);
template <> __device__ __forceinline__ void unpack16<SKV_F32>(const uint4& v, float* f) {
  f[0] = __uint_as_float(v.x), f[1] = __uint_as_float(v.y), f[2] = __uint_as_float(v.z), f[3] = __uint_as_float(v.w);
}
template <> __device__ __forceinline__ void unpack16<SKV_F16>(const uint4& v, float* f) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const half2v h = __builtin_bit_cast(half2v, w[i]);
    f[2 * i] = (float)h.x;
    f[2 * i + 1] = (float)h.y;
  }
}
template <> __device__ __forceinline__ void unpack16<SKV_BF16>(const uint4& v, float* f) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf16_lo(w[i]);
    f[2 * i + 1] = bf16_hi(w[i]);
  }
}

struct AddNormParams {
  const uint4* x;
  const uint4* y;  // NULL: no add
  const uint4* gamma;
  const uint4* beta;
  uint4* sum;      // NULL: sum not stored
  uint4* norm;
  int64_t ldx, ldy, lds, ldn;  // row strides in 16-byte vectors
  int32_t rows, vecs;          // vectors per row
  float eps, inv_n;
};

template <int DT, int VPL>
__global__ __launch_bounds__(256) void add_layernorm_kernel(AddNormParams p) {
  constexpr int EPL = Elt<DT>::EPL;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= p.rows) return;  // uniform over the wave
  float v[VPL][EPL];
  uint4 raw[VPL], gv[VPL], bv[VPL];
  // Every load up front (x, y, gamma, beta): one memory round trip per row.
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int c = lane + 64 * j;
    const bool in = c < p.vecs;
    raw[j] = in ? p.x[row * p.ldx + c] : make_uint4(0u, 0u, 0u, 0u);
    gv[j] = in ? p.gamma[c] : make_uint4(0u, 0u, 0u, 0u);
    bv[j] = in ? p.beta[c] : make_uint4(0u, 0u, 0u, 0u);
  }
  if (p.y) {
    uint4 ry[VPL];
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const int c = lane + 64 * j;
      ry[j] = c < p.vecs ? p.y[row * p.ldy + c] : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      float a[EPL], b[EPL];
      unpack16<DT>(raw[j], a);
      unpack16<DT>(ry[j], b);
#pragma unroll
      for (int e = 0; e < EPL; ++e) a[e] += b[e];
      raw[j] = pack16<DT>(a);  // rounded to the tensor type, like the stored sum
      const int c = lane + 64 * j;
      if (p.sum && c < p.vecs) p.sum[row * p.lds + c] = raw[j];
    }
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    unpack16<DT>(raw[j], v[j]);
#pragma unroll
    for (int e = 0; e < EPL; ++e) s += v[j][e];
  }
  const float mean = group_sum<64>(s) * p.inv_n;
  float q = 0.f;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    if (lane + 64 * j < p.vecs) {
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const float d = v[j][e] - mean;
        q = fmaf(d, d, q);
      }
    }
  }
  const float rstd = rsqrtf(group_sum<64>(q) * p.inv_n + p.eps);
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int c = lane + 64 * j;
    if (c >= p.vecs) continue;
    float g[EPL], b[EPL], o[EPL];
    unpack16<DT>(gv[j], g);
    unpack16<DT>(bv[j], b);
#pragma unroll
    for (int e = 0; e < EPL; ++e) o[e] = (v[j][e] - mean) * rstd * g[e] + b[e];
    p.norm[row * p.ldn + c] = pack16<DT>(o);
  }
}

template <int DT>
void launch_add_layernorm(const AddNormParams& p, int vpl, hipStream_t s) {
  const dim3 grid((uint32_t)cdiv(p.rows, 4));
  switch (vpl) {
    case 1: hipLaunchKernelGGL((add_layernorm_kernel<DT, 1>), grid, dim3(256), 0, s, p); break;
    case 2: hipLaunchKernelGGL((add_layernorm_kernel<DT, 2>), grid, dim3(256), 0, s, p); break;
    case 3: hipLaunchKernelGGL((add_layernorm_kernel<DT, 3>), grid, dim3(256), 0, s, p); break;
    case 4: hipLaunchKernelGGL((add_layernorm_kernel<DT, 4>), grid, dim3(256), 0, s, p); break;
    default: hipLaunchKernelGGL((add_layernorm_kernel<DT, 8>), grid, dim3(256), 0, s, p); break;
  }
}

// ---------------------------------------------------------------------------
// Multi-codebook embedding sum: out[r] = T_0[c_r0] + T_1[c_r1] + ... with every
// partial sum rounded to the tensor dtype, i.e. the bits of a sequential
// x = x + emb_k(codes[..., k]) in that dtype. One thread per 16-byte vector.
// ---------------------------------------------------------------------------
constexpr int kMaxCodebooks = 16;

struct EmbedSumParams {
  const int64_t* codes;
  int64_t codes_stride;  // elements between rows of codes
  const uint4* tables[kMaxCodebooks];
  uint4* out;
  int64_t out_stride;    // 16-byte vectors between output rows
  int64_t total;         // rows * vecs
  int32_t books, vocab, vecs;
};

template <int DT>
__global__ __launch_bounds__(256) void embed_sum_kernel(EmbedSumParams p) {
  constexpr int EPL = Elt<DT>::EPL;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= p.total) return;
  const int64_t r = idx / p.vecs;
  const int v = (int)(idx - r * p.vecs);
  uint4 raw[kMaxCodebooks];
#pragma unroll
  for (int k = 0; k < kMaxCodebooks; ++k) {  // every row load issues before the first add
    if (k < p.books) {
      const int64_t c = p.codes[r * p.codes_stride + k];
      raw[k] = (c >= 0 && c < p.vocab) ? p.tables[k][c * p.vecs + v] : make_uint4(0u, 0u, 0u, 0u);
    }
  }
  float acc[EPL], e[EPL];
  unpack16<DT>(raw[0], acc);
#pragma unroll
  for (int k = 1; k < kMaxCodebooks; ++k) {
    if (k < p.books) {
      unpack16<DT>(raw[k], e);
#pragma unroll
      for (int i = 0; i < EPL; ++i) acc[i] += e[i];
      unpack16<DT>(pack16<DT>(acc), acc);  // round the partial sum to the dtype
    }
  }
  p.out[r * p.out_stride + v] = pack16<DT>(acc);
}

// ---------------------------------------------------------------------------
// Attention.
// ---------------------------------------------------------------------------
#ifndef SKV_ATTN_WAVES
#define SKV_ATTN_WAVES 4
#endif
constexpr int kWaves = SKV_ATTN_WAVES;  // waves per attention workgroup
constexpr int kMaxChunkBlocks = 256;    // LDS block-id slots per chunk
constexpr int kPartPad = 4;             // partial record = m, l, pad, pad, acc[D]
// s_waitcnt immediate for vmcnt(0) alone (expcnt and lgkmcnt at their maxima).
constexpr int kWaitVmcnt0 = 0x0f70;
constexpr int kRankRows = 128;  // most rows a launch ranks by length (one or two per lane of a wave)
constexpr int kRankBits = 4;   // length bits the ranking orders by (16 length classes)

struct AttnParams {
  const uint4* q;  // strides below are in 16-byte vector units
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
  int32_t bs_shift;  // log2(bs) when bs is a power of two, else -1
  int64_t row_vecs;  // vectors per pool token row = Hkv * D / EPL
  // Byte size of each of the K and V regions the kernel may read: the pools
  // (paged) or one (slot, head) span of max_len keys (contiguous); the buffer
  // fast path needs it below kBufLimit.
  int64_t kv_bytes;
  // fused append (paged only): the Q newest keys of row b come from kn/vn
  // [B, Q, Hkv, D] and are written into the pool through the row's table.
  const uint4* kn;
  const uint4* vn;
  int64_t nsb, nsq, nsh;
  // contiguous addressing
  int64_t ss, sh, st;
  const int32_t* slots;
  // common
  const int32_t* lens;
  int32_t batch, qlen, heads, group, max_len, causal, chunk, nchunk_max;
  int32_t grid3d;  // grid (heads, rows, chunks) instead of (rows * heads, chunks)
  // Snake order (one chunk, grid3d): workgroup w of the dispatch order runs on
  // CU w mod 2^cu_shift while the grid fits one resident generation, so odd
  // rounds of 2^cu_shift workgroups take the (row, head) items in reverse; with
  // rows longest-first every CU then holds a mix of long and short rows.
  // row = umulhi(item, heads_magic), exact for items * heads < 2^32.
  int32_t snake, cu_shift;
  uint32_t items, heads_magic;
  // Rank order (paged, snake, q_len 1, at most kRankRows rows): item rows are ranks by length, so the
  // snake order balances the units' bytes whatever order the caller's rows come in.
  int32_t rank;
  float scale_log2;
  float* part;  // [rows*heads*nchunk_max][D + kPartPad]
};

#ifndef SKV_ATTN_UNROLL
#define SKV_ATTN_UNROLL 8  // most key rows a lane group loads before its math
#endif
#ifndef SKV_ATTN_SUB
#define SKV_ATTN_SUB 64  // most keys one wave loads per loop trip over contiguous K/V
#endif
// Paged K/V take shorter trips: a (row, head) ends with finer steps, which shortens
// the launch's tail (large-v3 batch 64: 14.97 -> 14.61 us, fp16 32 heads batch 64: 21.6 -> 21.3 us),
// while the contiguous cross-attention rows (1500 keys each) keep more rows in flight
// per lane (74.2 -> 73.4 us with 64-key trips). Both are powers of two, and 64 is a
// multiple of 32, so a chunk sized for the contiguous trip fits the paged one.
#ifndef SKV_ATTN_SUB_PAGED
#define SKV_ATTN_SUB_PAGED 32
#endif
template <int TPI, bool PAGED>
constexpr int unroll_for() {
  constexpr int sub = PAGED ? SKV_ATTN_SUB_PAGED : SKV_ATTN_SUB;
  return (sub / TPI) < 1 ? 1 : ((sub / TPI) > SKV_ATTN_UNROLL ? SKV_ATTN_UNROLL : (sub / TPI));
}

// Keys visible to query qi of batch row b.
__device__ __forceinline__ int visible_len(const AttnParams& p, int b, int qi) {
  int len = p.lens[b];
  if (p.causal) len -= (p.qlen - 1 - qi);
  len = len < 0 ? 0 : len;
  return len > p.max_len ? p.max_len : len;
}

// Merge the (m, l, acc) states of the TPI lane groups of a wave (lane offsets
// LPT, 2*LPT, ..., 32): the common maximum first, then plain sums of the
// rescaled l and acc. Every lane ends with the merged state of its dims.
template <int OFF>
__device__ __forceinline__ void max_steps(float& m) {
  if constexpr (OFF < 64) {
    m = fmaxf(m, xor_lane<OFF>(m));
    max_steps<OFF * 2>(m);
  }
}
template <int OFF, int N>
__device__ __forceinline__ void sum_steps(float& l, float* acc) {
  if constexpr (OFF < 64) {
    l += xor_lane<OFF>(l);
#pragma unroll
    for (int e = 0; e < N; ++e) acc[e] += xor_lane<OFF>(acc[e]);
    sum_steps<OFF * 2, N>(l, acc);
  }
}
template <int LPT, int EPL>
__device__ __forceinline__ void merge_groups(float& m, float& l, float* acc) {
  if constexpr (LPT < 64) {
    float mm = m;
    max_steps<LPT>(mm);
    const float s = __builtin_amdgcn_exp2f(m - (mm == kNegInf ? 0.f : mm));
    l *= s;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[e] *= s;
    sum_steps<LPT, EPL>(l, acc);
    m = mm;
  }
}

template <int DT>
__device__ __forceinline__ void write_out(const AttnParams& p, int64_t o_off, float l, const float* acc) {
  constexpr int EPL = Elt<DT>::EPL;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  float r[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) r[e] = acc[e] * inv;
  p.o[o_off] = pack16<DT>(r);
}

// 16 zero bytes: the load target of key slots that hold no key (past the
// row's length or behind an invalid block id), so every load is issued
// unconditionally and an empty slot contributes an exact zero.
__device__ __attribute__((aligned(16))) uint32_t g_zero16[4];

// One online-softmax step over N keys per lane group: scores from q.k (lane
// group sum), masked by ok when MASK (a trip whose keys are all present skips
// the selects), then the rescale and the p*v accumulation.
template <int DT, int LPT, int EPL, int N, bool MASK = true>
__device__ __forceinline__ void softmax_step(const uint4& qv, const uint4* kr, const uint4* vr, const bool* ok,
                                             float scale_log2, float& m, float& l, float* acc) {
  float sc[N];
  float mx = m;
#pragma unroll
  for (int u = 0; u < N; ++u) {
    const float d = group_sum<LPT>(dot16<DT>(qv, kr[u]));
    sc[u] = d * scale_log2;
    if constexpr (MASK) sc[u] = ok[u] ? sc[u] : kNegInf;
    mx = fmaxf(mx, sc[u]);
  }
  const float ref = (mx == kNegInf) ? 0.f : mx;
  const float alpha = __builtin_amdgcn_exp2f(m - ref);
  l *= alpha;
#pragma unroll
  for (int e = 0; e < EPL; ++e) acc[e] *= alpha;
#pragma unroll
  for (int u = 0; u < N; ++u) {
    const float pr = __builtin_amdgcn_exp2f(sc[u] - ref);
    l += pr;
    axpy16<DT>(pr, vr[u], acc);
  }
  m = mx;
}

// Buffer fast path: K/V are read with buffer loads against a descriptor of
// kv_bytes; an empty key slot gets an offset past that range, for which the
// hardware returns zeros, so loads need no data select and offsets are 32-bit.
constexpr int64_t kBufLimit = 0x7fffffff;

__device__ __forceinline__ uint4 load_buf(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kBufNt);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Grid: x = query row * heads + head, y = key chunk. FAST: the buffer path;
// for paged K/V it also needs a power-of-two block size (p.bs_shift) of at
// least TPI keys. Then the TPI keys one load instruction of a wave covers lie
// in one block, so each load's block id is wave-uniform: it is read from the
// block table with a scalar load, which travels through the scalar cache, not
// the CU's vector memory queue.
// The parameters of the prologue's address chain come first, as separate
// scalar arguments: the build preloads the first 14 argument dwords into
// scalar registers when the wave starts, so the chain's first memory access
// (block table, row length) does not wait for a kernel-argument load.
// qlen_group: q_len in bits 0-15, query heads per KV head in bits 16-31.
// flags: bit 0 grid3d, bit 1 snake order, bit 2 causal, bit 3 rank order, bits 8-15 cu_shift,
// bits 16-23 log2(block size) (the fast path's power-of-two block size).
// The paged variants are built for at least 5 waves per SIMD, the register
// budget of 5 resident workgroups per CU (a large decode batch's launch is one
// resident generation); at head_dim 64 they take 60-62 VGPRs.
template <int DT, int D, bool PAGED, bool FAST>
__global__ __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(PAGED ? 5 : 1))) void attention_kernel(
    const int32_t* __restrict__ a_tables, const int32_t* __restrict__ a_lens, const int32_t* __restrict__ a_trows,
    int32_t heads, int32_t tstride, int32_t max_len, int32_t chunk_len, uint32_t qlen_group, uint32_t flags,
    uint32_t items, uint32_t heads_magic, AttnParams p) {
  constexpr int EPL = Elt<DT>::EPL;
  constexpr int LPT = D / EPL;
  constexpr int TPI = 64 / LPT;
  constexpr int U = unroll_for<TPI, PAGED>();
  constexpr int SUB = TPI * U;
  constexpr int PSTRIDE = D + kPartPad;

  __shared__ int s_blk[PAGED ? kMaxChunkBlocks : 1];
  __shared__ float s_ml[kWaves][2];
  __shared__ float s_acc[kWaves][D];
  // Fast paged path: the fused-append K/V row, copied here by the load itself
  // (one 16-byte slot per lane of the last wave).
  __shared__ uint4 s_new[(PAGED && FAST) ? 2 : 1][64];
  __shared__ int s_ranked_row;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const uint32_t bx = blockIdx.x;
  const int qlen = (int)(qlen_group & 0xffffu), group = (int)(qlen_group >> 16);
  const bool causal = (flags >> 2) & 1u;
  const uint32_t cu_shift = (flags >> 8) & 0xffu;
  const int bs_shift = (int)((flags >> 16) & 0xffu);
  // Keys visible to query qi of a row whose cache holds row_len keys.
  auto visible = [&](int row_len, int qi) {
    int len = row_len;
    if (causal) len -= (qlen - 1 - qi);
    len = len < 0 ? 0 : len;
    return len > max_len ? max_len : len;
  };
  // Grid (heads, rows, chunks), or (rows * heads, chunks) when the rows exceed
  // the y limit. Every wave of a CU's resident workgroups runs this prologue on
  // the CU's one scalar unit before its first memory access, so the common
  // shapes (q_len 1, no KV grouping, one chunk) take no integer division.
  int h, row, chunk;
  int ranked_len = 0;  // rank order: the row's length, as the ranking read it
  if (flags & 2u) {
    const uint32_t w = bx + blockIdx.y * (uint32_t)heads;
    const uint32_t round = (1u << cu_shift) - 1u;
    const uint32_t base = w & ~round;
    uint32_t item = w;
    if ((w >> cu_shift) & 1u) {
      const uint32_t n = min(round + 1u, items - base);
      item = base + (n - 1u) - (w - base);
    }
    row = (int)__umulhi(item, heads_magic);
    h = (int)item - row * heads;
    chunk = 0;
    if constexpr (PAGED) {
      // Rank order: `row` is a rank, and the workgroup takes the row of that rank in the order of
      // the rows' length classes (the top kRankBits bits of the length below 2^bitlen(max_len):
      // longest first, ties to the lower row), which balances the units' bytes as well as an
      // exact sort to within one class. Every wave reads the lengths, one row per lane with a
      // buffer load (lanes past the batch read zero; the batch is items / heads, exact as for the
      // row above), and rows 64-127 with a second load when the batch has them. Rows already
      // longest-first need nothing more: the rank is the row. Otherwise wave 0 selects the row, a
      // radix selection over the class bits with wave ballots and then the rank's place within
      // its class, and hands it to the other waves through LDS. Batches of up to 64 rows take a
      // copy of this code without the second half.
      if (flags & 8u) {
        const uint32_t nrows = __umulhi(items, heads_magic);
        const __amdgpu_buffer_rsrc_t lres = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<int32_t*>(a_lens), (short)0, (int)(nrows * 4u), kBufWord3);
        const int lraw = (int)__builtin_amdgcn_raw_buffer_load_b32(lres, (uint32_t)lane * 4u, 0, 0);
        // The parameter-block fields of the address chain load while the lengths are in flight.
        asm volatile("" ::"s"(p.q), "s"(p.qsb), "s"(p.qsq), "s"(p.qsh), "s"(p.osb), "s"(p.osq), "s"(p.osh),
                     "s"(p.k), "s"(p.v), "s"(p.nb), "s"(p.row_vecs), "s"(p.kv_bytes), "s"(p.kn), "s"(p.vn),
                     "s"(p.nsb), "s"(p.nsh), "s"(p.nchunk_max));
        const int lenj = min(max(lraw, 0), max_len);
        auto rank = [&](auto two_c) __attribute__((always_inline)) {
          constexpr bool TWO = decltype(two_c)::value;  // rows 64-127 in a second register
          int lraw1 = 0, lenj1 = 0;
          if constexpr (TWO) {
            lraw1 = (int)__builtin_amdgcn_raw_buffer_load_b32(lres, (uint32_t)(lane + 64) * 4u, 0, 0);
            lenj1 = min(max(lraw1, 0), max_len);
          }
          const int prev = __shfl_up(lenj, 1);
          bool rises = lane > 0 && lenj > prev;  // the same in every wave (rows past the batch hold 0)
          if constexpr (TWO) {
            const int prev1 = __shfl_up(lenj1, 1);
            rises = rises || lenj1 > (lane == 0 ? __builtin_amdgcn_readlane(lenj, 63) : prev1);
          }
          if (__any(rises)) {
            if (__builtin_amdgcn_readfirstlane(wave) == 0) {
              uint64_t cand = __ballot((uint32_t)lane < nrows), cand1 = 0;
              if constexpr (TWO) cand1 = __ballot((uint32_t)lane + 64u < nrows);
              uint32_t k = (uint32_t)row;
              const int top = 31 - __clz(max(max_len, 1));
              for (int bit = top; bit >= max(top + 1 - kRankBits, 0); --bit) {
                const uint64_t ones = __ballot((lenj >> bit) & 1) & cand;
                uint64_t ones1 = 0;
                if constexpr (TWO) ones1 = __ballot((lenj1 >> bit) & 1) & cand1;
                const uint32_t c = (uint32_t)(__popcll(ones) + (TWO ? __popcll(ones1) : 0));
                if (k < c) {
                  cand = ones;
                  cand1 = ones1;
                } else {
                  k -= c;
                  cand &= ~ones;
                  cand1 &= ~ones1;
                }
              }
              // the k-th lowest row of the remaining class: rows 0-63 in cand, 64-127 in cand1
              int first = 0;
              if constexpr (TWO) {
                const uint32_t c0 = (uint32_t)__popcll(cand);
                if (k >= c0) {
                  k -= c0;
                  cand = cand1;
                  first = 64;
                }
              }
              for (; k > 0; --k) cand &= cand - 1;
              if (lane == 0) s_ranked_row = first + __ffsll((unsigned long long)cand) - 1;
            }
            lds_barrier();
            row = __builtin_amdgcn_readfirstlane(s_ranked_row);
          }
          if constexpr (TWO)
            ranked_len = row < 64 ? __builtin_amdgcn_readlane(lraw, row) : __builtin_amdgcn_readlane(lraw1, row - 64);
          else
            ranked_len = __builtin_amdgcn_readlane(lraw, row);
        };
        if (nrows > 64)
          rank(std::true_type{});
        else
          rank(std::false_type{});
      }
    }
  } else if (flags & 1u) {
    h = bx;
    row = blockIdx.y;
    chunk = blockIdx.z;
  } else {
    row = bx / heads;
    h = bx - row * heads;
    chunk = blockIdx.y;
  }
  const int rh = row * heads + h;
  int b = row, qi = 0;
  if (qlen != 1) {
    b = row / qlen;
    qi = row - b * qlen;
  }
  const int g = lane / LPT;
  const int j = lane - g * LPT;
  const int64_t o_off = (int64_t)b * p.osb + (int64_t)qi * p.osq + (int64_t)h * p.osh + j;
  const int t_begin = chunk * chunk_len;
  const int kvh = group == 1 ? h : h / group;
  const uint4* zero = reinterpret_cast<const uint4*>(g_zero16);

  // Loads in the order of the address chain. First one scalar batch: the row
  // length, the table row and the parameter-block fields used before the
  // first K/V load. The empty asm takes them as scalar-register operands, so
  // every one of these loads issues before a single wait (left to itself the
  // compiler issues each where it is first used and waits for each in turn).
  // The asm has no memory effects, so the loads behind it keep their scalar
  // form. Then (general path) the chunk's block ids, staged in LDS for the
  // workgroup, then q and the fused-append row, which are first needed after
  // the first K/V loads have been issued. Block ids are staged for the chunk's
  // span up to max_len (inside the table row, which covers max_len), so the
  // staging does not wait for the row length. The fast path reads block ids
  // per wave with scalar loads in its key loop instead.
  int row_len = PAGED && (flags & 8u) ? ranked_len : a_lens[b];
  const int trow = PAGED && a_trows ? a_trows[b] : b;
  asm("" : "+s"(row_len)
      : "s"(trow), "s"(p.q), "s"(p.qsb), "s"(p.qsq), "s"(p.qsh), "s"(p.osb), "s"(p.osq), "s"(p.osh),
        "s"(p.k), "s"(p.v), "s"(p.nb), "s"(p.row_vecs), "s"(p.kv_bytes), "s"(p.kn), "s"(p.vn),
        "s"(p.nsb), "s"(p.nsh), "s"(p.nchunk_max));
  const int len = visible(row_len, qi);
  int first_blk = 0;
  const int32_t* tbl = nullptr;
  if constexpr (PAGED) {
    tbl = a_tables + (int64_t)trow * tstride;
    if constexpr (!FAST) {
      const int span_end = min(t_begin + chunk_len, max_len);
      first_blk = t_begin / p.bs;
      const int last_blk = (span_end - 1) / p.bs;
      const int nblk = span_end > t_begin ? last_blk - first_blk + 1 : 0;
      for (int i = threadIdx.x; i < nblk; i += 64 * kWaves) {
        const int blk = tbl[first_blk + i];
        s_blk[i] = ((uint32_t)blk < (uint32_t)p.nb) ? blk : -1;
      }
    }
  }
  // Block id of key t from the table row (fast path), -1 when invalid.
  auto table_block = [&](int t) {
    const int blk = tbl[t >> bs_shift];
    return ((uint32_t)blk < (uint32_t)p.nb) ? blk : -1;
  };
  const uint4 qv = p.q[(int64_t)b * p.qsb + (int64_t)qi * p.qsq + (int64_t)h * p.qsh + j];
  // A fused append of one key (q_len 1, the decode step): the last wave loads
  // the new K/V row, scores it and writes it to the pool, so the append adds no
  // memory round trip. Its kn/vn address does not depend on the row length.
  // The general path loads it here, into registers, and scores it before the
  // pool loop; the fast paged path copies it into LDS at the start of the last
  // wave's pool trips (no registers held across them) and scores it after them.
  const bool one_new = PAGED && p.kn && qlen == 1;
  const int64_t new_off = (int64_t)b * p.nsb + (int64_t)kvh * p.nsh + j;
  uint4 nk = make_uint4(0u, 0u, 0u, 0u), nv = nk;
  if constexpr (!(PAGED && FAST)) {
    if (one_new && wave == kWaves - 1 && g == 0) {
      nk = p.kn[new_off];
      nv = p.vn[new_off];
    }
  }

  if (len == 0) {
    if (chunk == 0 && wave == 0 && g == 0) p.o[o_off] = make_uint4(0u, 0u, 0u, 0u);
    return;
  }
  const int nchunks = p.nchunk_max == 1 ? 1 : (len + chunk_len - 1) / chunk_len;
  if (chunk >= nchunks) return;  // uniform over the workgroup
  const int t_end = min(t_begin + chunk_len, len);

  // Keys [t_begin, pool_end) are read from K/V; with a fused append the
  // newest keys [new_begin, len) come from kn/vn instead (fresh loop below).
  int pool_end = t_end;
  int new_begin = t_end;
  int64_t base = 0;
  float m = kNegInf, l = 0.f;
  float acc[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) acc[e] = 0.f;
  // Fused append of one key: the new key is len - 1; the chunk that holds it
  // (uniform test) scores it in the last wave, and the first head of each KV
  // group stores it into the pool. The fast path reads the destination's
  // table entry before its pool trips (app_raw), so the store at the end of
  // the wave does not wait for a table read.
  uint32_t app_raw = ~0u;  // raw table entry; checked where it is used
  auto score_new_key = [&]() {
    if (new_begin >= t_begin && new_begin < t_end && wave == kWaves - 1) {
      if constexpr (PAGED && FAST) {
        if (g == 0) {  // the LDS copy has landed (the caller waited for it)
          nk = s_new[0][lane];
          nv = s_new[1][lane];
        }
      }
      const bool ok[1] = {g == 0};
      softmax_step<DT, LPT, EPL, 1>(qv, &nk, &nv, ok, p.scale_log2, m, l, acc);
      if (g == 0 && (group == 1 || h % group == 0)) {
        const int bi = FAST ? new_begin >> bs_shift : new_begin / p.bs;
        const int blk = FAST ? (app_raw < (uint32_t)p.nb ? (int)app_raw : -1) : s_blk[bi - first_blk];
        if (blk >= 0) {
          const int64_t dst = ((int64_t)blk * p.bs + (new_begin - bi * p.bs)) * p.row_vecs + base;
          const_cast<uint4*>(p.k)[dst] = nk;
          const_cast<uint4*>(p.v)[dst] = nv;
        }
      }
    }
  };
  if constexpr (PAGED) {
    if constexpr (!FAST) __syncthreads();
    base = (int64_t)kvh * LPT + j;
    if (p.kn) {
      new_begin = visible(row_len, qlen - 1) - qlen;
      pool_end = max(t_begin, min(new_begin, t_end));
    }
    if (one_new) {
      // The fast path scores the new key after its first K/V loads are issued.
      if constexpr (!FAST) score_new_key();
    } else if (p.kn) {
      // Append: the last query row's workgroups of the first head of each KV
      // group write the new keys of their chunk into the pool.
      if (qi == qlen - 1 && h % group == 0) {
        const int w0 = max(new_begin, t_begin);
        const int nw = t_end - w0;
        for (int i = threadIdx.x; i < 2 * nw * LPT; i += 64 * kWaves) {
          const int kv = i >= nw * LPT;
          const int r = i - kv * nw * LPT;
          const int tt = w0 + r / LPT;
          const int jj = r - (r / LPT) * LPT;
          const int bi = tt / p.bs;
          const int blk = FAST ? table_block(tt) : s_blk[bi - first_blk];
          if (blk >= 0) {
            const int64_t dst = ((int64_t)blk * p.bs + (tt - bi * p.bs)) * p.row_vecs + (int64_t)kvh * LPT + jj;
            const int64_t src = (int64_t)b * p.nsb + (int64_t)(tt - new_begin) * p.nsq + (int64_t)kvh * p.nsh + jj;
            uint4* pool = const_cast<uint4*>(kv ? p.v : p.k);
            pool[dst] = (kv ? p.vn : p.kn)[src];
          }
        }
      }
    }
  } else {
    const int slot = p.slots ? p.slots[b] : b;
    base = (int64_t)slot * p.ss + (int64_t)kvh * p.sh + j;
  }

  if constexpr (FAST) {
    // 32-bit byte offsets against per-launch (paged) or per-workgroup (contiguous) descriptors.
    const char* kb = reinterpret_cast<const char*>(p.k);
    const char* vb = reinterpret_cast<const char*>(p.v);
    if constexpr (!PAGED) {  // descriptor base: the workgroup's (slot, head) span
      kb += (base - j) * 16;
      vb += (base - j) * 16;
    }
    const __amdgpu_buffer_rsrc_t kres = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(kb), (short)0,
                                                                          (int)p.kv_bytes, kBufWord3);
    const __amdgpu_buffer_rsrc_t vres = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(vb), (short)0,
                                                                          (int)p.kv_bytes, kBufWord3);
    const uint32_t row_bytes = PAGED ? (uint32_t)p.row_vecs * 16u : (uint32_t)p.st * 16u;
    const uint32_t col_bytes = PAGED ? (uint32_t)base * 16u : (uint32_t)j * 16u;
    // Wave-uniform start, so the paged path's table reads are scalar loads.
    const int s0 = t_begin + __builtin_amdgcn_readfirstlane(wave) * SUB;
    if constexpr (PAGED) {
      const uint32_t lane_off = (uint32_t)g * row_bytes + col_bytes;
      const uint32_t bmask = (1u << bs_shift) - 1u;
      const uint32_t blk_bytes = row_bytes << bs_shift;
      const uint32_t last_key = (uint32_t)pool_end - 1u;
      const uint32_t* trow = reinterpret_cast<const uint32_t*>(tbl);
      uint32_t cu_off[U];  // ((u*TPI) & bmask) * row_bytes, wave-uniform
#pragma unroll
      for (int u = 0; u < U; ++u) cu_off[u] = ((uint32_t)(u * TPI) & bmask) * row_bytes;
      // Keys s + u*TPI .. s + u*TPI + TPI - 1 lie in one block, at position
      // (s & bmask) + ((u*TPI) & bmask) + g: s is a multiple of SUB, and the
      // block size and SUB are powers of two with TPI <= block size. A load
      // wholly past pool_end reads the last key's table entry and masks every
      // lane. All table loads of a trip issue before the first use, so the trip
      // waits for one scalar round trip. A trip whose SUB keys all lie before
      // pool_end in valid blocks (every trip of a row but its last, unless an
      // id is invalid) takes a copy of the loads and math without per-lane
      // masks; the test is on scalar values, so the branch is wave-uniform.
      auto trip_body = [&](auto clean_c, int s, const uint32_t* raw, uint32_t trip_off) __attribute__((always_inline)) {
        constexpr bool CLEAN = decltype(clean_c)::value;
        uint4 kr[U], vr[U];
        uint32_t voff[U];
        bool ok[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const uint32_t sb = raw[u] * blk_bytes + trip_off + cu_off[u];
          if constexpr (CLEAN) {
            voff[u] = lane_off + sb;
            ok[u] = true;
          } else {
            const bool valid = raw[u] < (uint32_t)p.nb && g < pool_end - (s + u * TPI);
            voff[u] = (lane_off + sb) | (valid ? 0u : kBufOutOfRange);
            ok[u] = valid;
          }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) kr[u] = load_buf(kres, voff[u]);
#pragma unroll
        for (int u = 0; u < U; ++u) vr[u] = load_buf(vres, voff[u]);
        // Keep all 2*U loads in flight before the math: without this fence
        // the scheduler may sink loads into the math to save registers,
        // which serialises the memory latency.
        __builtin_amdgcn_sched_barrier(0);
        softmax_step<DT, LPT, EPL, U, !CLEAN>(qv, kr, vr, ok, p.scale_log2, m, l, acc);
      };
      auto trip = [&](int s) __attribute__((always_inline)) {
        uint32_t raw[U];
#pragma unroll
        for (int u = 0; u < U; ++u) raw[u] = trow[min((uint32_t)(s + u * TPI), last_key) >> bs_shift];
        __builtin_amdgcn_sched_barrier(0);
        const uint32_t trip_off = ((uint32_t)s & bmask) * row_bytes;
        bool blocks_ok = true;
#pragma unroll
        for (int u = 0; u < U; ++u) blocks_ok = blocks_ok && raw[u] < (uint32_t)p.nb;
        if (blocks_ok && s + SUB <= pool_end)
          trip_body(std::true_type{}, s, raw, trip_off);
        else
          trip_body(std::false_type{}, s, raw, trip_off);
      };
      // No load of this wave is waited for before its first K/V loads issue.
      // The last wave's pool trips are a separate copy of the loop: while the
      // LDS copy of the new key's row is outstanding, the compiler waits for
      // all of a trip's loads before its first use, so only that copy carries
      // it and the other waves' math starts on a trip's first load.
      auto pool_trips = [&](auto last_wave) {
        if constexpr (decltype(last_wave)::value) {
          if (one_new && g == 0) {
            using lds_ptr = __attribute__((address_space(3))) void*;
            using glb_ptr = __attribute__((address_space(1))) void*;
            __builtin_amdgcn_global_load_lds((glb_ptr)(p.kn + new_off), (lds_ptr)&s_new[0][0], 16, 0, 0);
            __builtin_amdgcn_global_load_lds((glb_ptr)(p.vn + new_off), (lds_ptr)&s_new[1][0], 16, 0, 0);
          }
          if (one_new) app_raw = (uint32_t)tbl[new_begin >> bs_shift];
        }
        for (int s = s0; s < pool_end; s += kWaves * SUB) trip(s);
        if constexpr (decltype(last_wave)::value) {
          if (one_new) {
            // The LDS copy has landed once this wave's loads have all completed; wait
            // for it whether or not this chunk scores the new key, so no copy is in
            // flight when the workgroup ends.
            __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
            score_new_key();
          }
        }
      };
      if (__builtin_amdgcn_readfirstlane(wave) == kWaves - 1)
        pool_trips(std::true_type{});
      else
        pool_trips(std::false_type{});
    } else {
      for (int s = s0; s < pool_end; s += kWaves * SUB) {
        uint32_t off[U];
        bool ok[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int t = s + u * TPI + g;
          const bool valid = t < pool_end;
          off[u] = valid ? (uint32_t)t * row_bytes + col_bytes : kBufOutOfRange;
          ok[u] = valid;
        }
        uint4 kr[U], vr[U];
#pragma unroll
        for (int u = 0; u < U; ++u) kr[u] = load_buf(kres, off[u]);
#pragma unroll
        for (int u = 0; u < U; ++u) vr[u] = load_buf(vres, off[u]);
        __builtin_amdgcn_sched_barrier(0);
        softmax_step<DT, LPT, EPL, U>(qv, kr, vr, ok, p.scale_log2, m, l, acc);
      }
    }
  } else {
    for (int s = t_begin + wave * SUB; s < pool_end; s += kWaves * SUB) {
      const uint4* kp[U];
      const uint4* vp[U];
      bool ok[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int t = s + u * TPI + g;
        bool valid = t < pool_end;
        int64_t off;
        if constexpr (PAGED) {
          const int bi = t / p.bs;
          const int blk = s_blk[min(bi - first_blk, kMaxChunkBlocks - 1)];
          valid = valid && blk >= 0;
          off = ((int64_t)blk * p.bs + (t - bi * p.bs)) * p.row_vecs + base;
        } else {
          off = base + (int64_t)t * p.st;
        }
        kp[u] = valid ? p.k + off : zero;
        vp[u] = valid ? p.v + off : zero;
        ok[u] = valid;
      }
      uint4 kr[U], vr[U];
#pragma unroll
      for (int u = 0; u < U; ++u) kr[u] = load_stream(kp[u]);
#pragma unroll
      for (int u = 0; u < U; ++u) vr[u] = load_stream(vp[u]);
      __builtin_amdgcn_sched_barrier(0);
      softmax_step<DT, LPT, EPL, U>(qv, kr, vr, ok, p.scale_log2, m, l, acc);
    }
  }

  if constexpr (PAGED) {
    // Fresh keys of a fused append with q_len > 1: one per lane group.
    if (!one_new && new_begin < t_end) {
      const int64_t nbase = (int64_t)b * p.nsb + (int64_t)kvh * p.nsh + j;
      for (int s = max(t_begin, new_begin) + wave * TPI; s < t_end; s += kWaves * TPI) {
        const int t = s + g;
        bool ok[1] = {t < t_end};
        const int64_t off = nbase + (int64_t)(t - new_begin) * p.nsq;
        const uint4 kr[1] = {load_stream(ok[0] ? p.kn + off : zero)};
        const uint4 vr[1] = {load_stream(ok[0] ? p.vn + off : zero)};
        softmax_step<DT, LPT, EPL, 1>(qv, kr, vr, ok, p.scale_log2, m, l, acc);
      }
    }
  }

  if constexpr (LPT == 8 && EPL == 8) {
    // Head dim 64 in fp16/bf16: the 8 lane groups (lanes 8g + j, dims 8j .. 8j + 7)
    // move to their common maximum, then the sums are reduce-scattered rather
    // than all-reduced: the permlane32 and permlane16 swaps exchange half of
    // the remaining elements each (a swap of two different registers hands
    // each half-wave or row the partner's copy of the element it keeps), and a
    // DPP step within each row the last one, so lane (g, j) ends with dim
    // 8j + g summed over the groups. Wave 0 then merges the 4 waves with one
    // dim per lane.
    float mm = m;
    max_steps<8>(mm);
    const float gs = __builtin_amdgcn_exp2f(m - (mm == kNegInf ? 0.f : mm));
    l *= gs;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] *= gs;
    l += xor_lane<8>(l);
    l += xor_lane<16>(l);
    l += xor_lane<32>(l);
    float r1[4], r2[2];
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // lanes 0-31 keep element i, lanes 32-63 element i + 4
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[i]), __float_as_uint(acc[i + 4]), false,
                                                       false);
      r1[i] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {  // row R of 16 lanes keeps element i + 2R
      const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(r1[i]), __float_as_uint(r1[i + 2]), false,
                                                       false);
      r2[i] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
    const bool odd = (lane & 8) != 0;  // lane (g, j) keeps element g
    const float keep = odd ? r2[1] : r2[0];
    const float send = odd ? r2[0] : r2[1];
    const float fin = keep + xor_lane<8>(send);
    s_acc[wave][8 * j + g] = fin;
    if (lane == 0) {
      s_ml[wave][0] = mm;
      s_ml[wave][1] = l;
    }
    __syncthreads();
    if (wave != 0) return;
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_ml[w][0]);
    const float ref = M == kNegInf ? 0.f : M;
    float L = 0.f, A = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float ew = __builtin_amdgcn_exp2f(s_ml[w][0] - ref);
      L += ew * s_ml[w][1];
      A += ew * s_acc[w][lane];
    }
    const int64_t o_row = o_off - j;  // the (row, head)'s first 16-byte vector of the output
    if (nchunks == 1) {
      const float r = L > 0.f ? A * (1.f / L) : 0.f;
      const uint32_t bits = DT == SKV_BF16 ? f32_to_bf16_bits(r) : (pack_half2(r, 0.f) & 0xffffu);
      reinterpret_cast<uint16_t*>(p.o + o_row)[lane] = (uint16_t)bits;
      return;
    }
    float* rec = p.part + ((int64_t)rh * p.nchunk_max + chunk) * PSTRIDE;
    rec[kPartPad + lane] = A;
    if (lane == 0) *reinterpret_cast<float2*>(rec) = make_float2(M, L);
    return;
  } else {
    merge_groups<LPT, EPL>(m, l, acc);

    // Merge the kWaves wave states through LDS.
    if (g == 0) {
#pragma unroll
      for (int e = 0; e < EPL; ++e) s_acc[wave][j * EPL + e] = acc[e];
      if (j == 0) {
        s_ml[wave][0] = m;
        s_ml[wave][1] = l;
      }
    }
    __syncthreads();
    if (wave != 0 || g != 0) return;
    float M = s_ml[0][0], L = s_ml[0][1];
    float A[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) A[e] = s_acc[0][j * EPL + e];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) merge_state<EPL>(M, L, A, s_ml[w][0], s_ml[w][1], &s_acc[w][j * EPL]);

    if (nchunks == 1) {
      write_out<DT>(p, o_off, L, A);
      return;
    }
    float* rec = p.part + ((int64_t)rh * p.nchunk_max + chunk) * PSTRIDE;
    float4* dst = reinterpret_cast<float4*>(rec + kPartPad + j * EPL);
#pragma unroll
    for (int e = 0; e < EPL; e += 4) dst[e / 4] = make_float4(A[e], A[e + 1], A[e + 2], A[e + 3]);
    if (j == 0) *reinterpret_cast<float2*>(rec) = make_float2(M, L);
  }
}

// Combine the per-chunk partials of rows that span more than one chunk.
// One wave per (row, head); lane group g folds chunks g, g + TPI, ...
template <int DT, int D>
__global__ __launch_bounds__(256) void merge_kernel(AttnParams p) {
  constexpr int EPL = Elt<DT>::EPL;
  constexpr int LPT = D / EPL;
  constexpr int TPI = 64 / LPT;
  constexpr int PSTRIDE = D + kPartPad;
  const int lane = threadIdx.x & 63;
  const int64_t rh = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int32_t rows = p.batch * p.qlen;
  if (rh >= (int64_t)rows * p.heads) return;
  const int row = (int)(rh / p.heads);
  const int h = (int)(rh - (int64_t)row * p.heads);
  const int b = row / p.qlen;
  const int qi = row - b * p.qlen;
  const int len = visible_len(p, b, qi);
  const int nchunks = (len + p.chunk - 1) / p.chunk;
  if (nchunks <= 1) return;
  const int g = lane / LPT;
  const int j = lane - g * LPT;
  float M = kNegInf, L = 0.f;
  float A[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) A[e] = 0.f;
  const float* part = p.part + rh * p.nchunk_max * PSTRIDE;
  for (int c = g; c < nchunks; c += TPI) {
    const float* rec = part + (int64_t)c * PSTRIDE;
    const float2 ml = *reinterpret_cast<const float2*>(rec);
    const float4* src = reinterpret_cast<const float4*>(rec + kPartPad + j * EPL);
    float ac[EPL];
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
  if (g == 0) write_out<DT>(p, (int64_t)b * p.osb + (int64_t)qi * p.osq + (int64_t)h * p.osh + j, L, A);
}

// ---------------------------------------------------------------------------
// Multi-query attention over contiguous K/V on the matrix cores (cross-attention
// of a prompt, q_len >= 2, non-causal, head_dim 64, fp16/bf16).
//
// One workgroup of kWaves waves owns one (row, head, tile of 16 queries, key
// chunk): the tile's queries share every K/V load, so K/V are read once per tile
// instead of once per query. Per 32 keys a wave runs
//   S^T[32 keys x 16 q] = K . Q^T   4 x v_mfma_f32_16x16x32 (2 key tiles x 2 dim slabs)
//   O^T[64 d x 16 q]   += V^T . P^T  4 x v_mfma_f32_16x16x32 (4 dim blocks)
// with the gfx950 16x16x32 layouts: operand lane l holds row/column l % 16 and
// 8 contraction elements for lane group g = l / 16; result lane l holds rows
// 4g .. 4g+3 of column l % 16. The contraction index an element stands for only
// has to agree between the two operands, so
//   * K is loaded as it lies (lane: key 16t + l%16, dims 32s + 8g .. +8);
//   * S^T's result gives lane l the scores of query l%16 for keys 4g+i (tile 0)
//     and 16+4g+i (tile 1): exactly the 8 keys {K_g} it contributes to P^T;
//   * V^T needs 8 keys of one dim per lane: the gfx950 transpose load
//     (ds_read_b64_tr_b16) reads them from the row-major LDS rows of the keys
//     (vt_operand), two loads of 4 keys per operand.
// Online softmax per query (base 2), the max over a 32-key step reduced across
// the 4 lane groups. P enters its product with V in the input dtype: fp16 rounds
// it once (the row sums then add the rounded values, so the weights stay a convex
// combination); bf16 adds the product of the rounded remainder, which keeps the
// weights to ~16 bits.
// The waves merge through LDS; a split row writes per-query partials that
// merge_kernel combines.
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int DT>
__device__ __forceinline__ f32x4 mfma_16x16x32(const uint4& a, const uint4& b, const f32x4& c) {
  if constexpr (DT == SKV_BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  }
}

// Two fp32 values rounded to the dtype (to nearest even) and packed, first value in the
// low half: v_cvt_pk_bf16_f32 / v_cvt_pk_f16 style conversions, no branches.
template <int DT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  const f32x2 f = {a, b};
  if constexpr (DT == SKV_BF16) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf162v));
  } else {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, half2v));
  }
}
template <int DT>
__device__ __forceinline__ float lo16(uint32_t w) {
  if constexpr (DT == SKV_BF16) {
    return bf16_lo(w);
  } else {
    return (float)__builtin_bit_cast(half2v, w).x;
  }
}
template <int DT>
__device__ __forceinline__ float hi16(uint32_t w) {
  if constexpr (DT == SKV_BF16) {
    return bf16_hi(w);
  } else {
    return (float)__builtin_bit_cast(half2v, w).y;
  }
}

// V^T operand of one 16-dim block straight from row-major LDS rows with the gfx950
// transpose load ds_read_b64_tr_b16. Within each 16-lane group, element j of lane i's
// result is element i % 4 of the 8-byte chunk addressed by lane 4j + i / 4 of the group
// (checked on the GPU). Lane 4kk + q of group g addresses key K_g[kk] (first load) and
// K_g[4 + kk] (second load), dims 16 db + 4q .. +3, with K_g = {4g .. 4g+3, 16+4g ..
// 16+4g+3}: lane (g, m) then holds dim 16 db + m of the keys K_g in that order, the k
// order of the P^T operand. row_a / row_b: this lane's two chunk addresses for db = 0.
typedef short v4i16 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 vt_operand(const char* row_a, const char* row_b, int db) {
  typedef __attribute__((address_space(3))) v4i16* lds_v4;
  const v4i16 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4)(const_cast<char*>(row_a) + 32 * db));
  const v4i16 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4)(const_cast<char*>(row_b) + 32 * db));
  const uint2 ua = __builtin_bit_cast(uint2, a), ub = __builtin_bit_cast(uint2, b);
  return make_uint4(ua.x, ua.y, ub.x, ub.y);
}

constexpr int kMqQueries = 16;  // queries per tile (the MFMA's N)
// Lazy rescaling of the matrix-core kernels' online softmax: a wave's reference maximum
// (and with it the accumulators' scale) moves only when some query's step maximum exceeds it
// by more than this (log2 units), so the weights stay below 2^8, which the fp32 sums and the
// fp16/bf16 P operands hold at unchanged relative precision. With 16 queries per wave some
// query's maximum grows in most steps: rescaling at every growth multiplied the accumulators
// almost every step.
constexpr float kLazyMaxLog2 = 8.f;
static_assert(kWaves == 4, "mq_attention_kernel: each of the 4 waves finalises one 16-dim block");

// 3 waves per SIMD: the register budget that holds the next step's loads in flight without
// spilling (4 spills and halves the rate; 2 is no faster).
// PAGED: K/V come from the block pools through the row's table (power-of-two block size of
// at least 8 keys, so the 8 keys of one load instruction share a block id, read with a
// scalar load); otherwise from the contiguous [slot, head, T, D] layout.
template <int DT, bool PAGED>
__global__ __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(3))) void
mq_attention_kernel(AttnParams p, int32_t qtiles) {
  constexpr int D = 64;
  constexpr int PSTRIDE = D + kPartPad;
  __shared__ float s_m[kWaves][kMqQueries];
  __shared__ float s_l[kWaves][kMqQueries];
  // Per-wave K/V staging rows during the key loop; the wave merge reuses the space.
  constexpr int kStageBytes = kWaves * 2 * 32 * (D * 2 + 16);
  static_assert(kStageBytes >= (int)sizeof(float) * kWaves * kMqQueries * (D + 4), "merge buffer fits the staging");
  __shared__ __attribute__((aligned(16))) char s_stage[kStageBytes];
  auto s_acc = reinterpret_cast<float (*)[kMqQueries][D + 4]>(s_stage);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));  // wave-uniform
  const int g = lane >> 4;   // lane group of the MFMA layouts
  const int n = lane & 15;   // query column (result, P^T) / key or dim row (operands)
  const int h = (int)(blockIdx.x % (uint32_t)p.heads);
  const int qt = (int)(blockIdx.x / (uint32_t)p.heads);
  const int b = blockIdx.y;
  const int chunk = blockIdx.z;
  const int kvh = p.group == 1 ? h : h / p.group;

  int len = p.lens[b];
  len = len < 0 ? 0 : (len > p.max_len ? p.max_len : len);
  const int qi = qt * kMqQueries + n;  // this lane's query (result layout)
  const bool q_ok = qi < p.qlen;
  if (len == 0) {
    if (chunk == 0 && wave < 4 && q_ok) {  // zero output: lane writes dims 16*wave + 4g .. +4
      uint2* o = reinterpret_cast<uint2*>(p.o + (int64_t)b * p.osb + (int64_t)qi * p.osq + (int64_t)h * p.osh);
      o[(16 * wave + 4 * g) / 4] = make_uint2(0u, 0u);
    }
    return;
  }
  const int nchunks = p.nchunk_max == 1 ? 1 : (len + p.chunk - 1) / p.chunk;
  if (chunk >= nchunks) return;
  const int t_begin = chunk * p.chunk;
  const int t_end = min(t_begin + p.chunk, len);

  // Q^T operand: lane (query n, group g) holds dims 32s + 8g .. +8 for slabs s = 0, 1.
  uint4 qf[2];
#pragma unroll
  for (int sl = 0; sl < 2; ++sl) {
    qf[sl] = make_uint4(0u, 0u, 0u, 0u);
    if (q_ok) qf[sl] = p.q[(int64_t)b * p.qsb + (int64_t)qi * p.qsq + (int64_t)h * p.qsh + sl * 4 + g];
  }

  // Descriptors over the row's (slot, head) span (contiguous) or over the whole pool (paged).
  const char* kb = reinterpret_cast<const char*>(p.k);
  const char* vb = reinterpret_cast<const char*>(p.v);
  uint32_t row_bytes, col_base = 0;
  const uint32_t* trow = nullptr;
  if constexpr (PAGED) {
    row_bytes = (uint32_t)p.row_vecs * 16u;
    col_base = (uint32_t)kvh * (uint32_t)(D * 2);
    trow = reinterpret_cast<const uint32_t*>(p.tables + (int64_t)(p.trows ? p.trows[b] : b) * p.tstride);
  } else {
    const int slot = p.slots ? p.slots[b] : b;
    kb += ((int64_t)slot * p.ss + (int64_t)kvh * p.sh) * 16;
    vb += ((int64_t)slot * p.ss + (int64_t)kvh * p.sh) * 16;
    row_bytes = (uint32_t)p.st * 16u;
  }
  const __amdgpu_buffer_rsrc_t kres =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(kb), (short)0, (int)p.kv_bytes, kBufWord3);
  const __amdgpu_buffer_rsrc_t vres =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(vb), (short)0, (int)p.kv_bytes, kBufWord3);
  // Byte offset of key `key` (its row's column base added), out of range past t_end or
  // behind an invalid block id. key0 is the wave-uniform first key of a load instruction;
  // blk_ok reports (wave-uniformly) whether those 8 keys have a valid block.
  auto key_offset = [&](int key0, int key, bool& blk_ok) -> uint32_t {
    if constexpr (PAGED) {
      // Clamped to the last key so the table index stays inside the row (which covers max_len).
      const uint32_t k0 = (uint32_t)__builtin_amdgcn_readfirstlane(min(key0, t_end - 1));
      const uint32_t blk = trow[k0 >> p.bs_shift];  // wave-uniform: a scalar load
      blk_ok = blk < (uint32_t)p.nb;
      return key < t_end && blk_ok
                 ? (blk * (uint32_t)p.bs + ((uint32_t)key & ((uint32_t)p.bs - 1u))) * row_bytes + col_base
                 : kBufOutOfRange;
    } else {
      blk_ok = true;
      return key < t_end ? (uint32_t)key * row_bytes : kBufOutOfRange;
    }
  };
  // V^T operand chunks (vt_operand): lane 4kk + q of group g reads keys K_g[kk] and
  // K_g[4 + kk], dims 16 db + 4q .. +3.
  const int vt_key = 4 * g + ((lane & 15) >> 2);
  const int vt_col = 8 * (lane & 3);

  float m = kNegInf, l = 0.f;  // this lane's query n; l sums the keys of this lane group
  float ref = 0.f;             // m, or 0 while m is -inf: the exponents' offset
  f32x4 acc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};

  constexpr int STEP = 32;  // keys per MFMA step; waves take steps in turn
  // Loads read whole 128-byte key rows (8 lanes per row, 8 rows per instruction) and go
  // through this wave's LDS rows (padded to 144 bytes) to reach the operand layouts: the
  // operands want 16 different keys in every 16 lanes, which as direct loads would touch
  // 16 cache lines per pass.
  constexpr int kRowPad = D * 2 + 16;
  char* lds_k = s_stage + wave * (2 * STEP * kRowPad);
  char* lds_v = lds_k + STEP * kRowPad;
  const int nat_row = lane >> 3, nat_col = (lane & 7) * 16;  // key row / byte column of a load
  // Returns the step's valid-key mask (bit j: key base + j lies in a valid block).
  auto load_step = [&](int base, uint4 (&kr)[4], uint4 (&vr)[4]) -> uint32_t {
    uint32_t off[4], mask = 0u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      bool blk_ok;
      const uint32_t o = key_offset(base + 8 * i, base + 8 * i + nat_row, blk_ok);
      off[i] = o == kBufOutOfRange ? o : o + (uint32_t)nat_col;
      mask |= blk_ok ? 0xffu << (8 * i) : 0u;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      kr[i] = load_buf(kres, off[i]);
      vr[i] = load_buf(vres, off[i]);
    }
    return mask;
  };
  auto compute_step = [&](int base, const uint4 (&kr)[4], const uint4 (&vr)[4], uint32_t mask) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *reinterpret_cast<uint4*>(lds_k + (8 * i + nat_row) * kRowPad + nat_col) = kr[i];
      *reinterpret_cast<uint4*>(lds_v + (8 * i + nat_row) * kRowPad + nat_col) = vr[i];
    }
    __builtin_amdgcn_wave_barrier();
    // K operand of tile t, slab s: key 16t + n, dims 32s + 8g .. +8.
    f32x4 sc[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const char* row = lds_k + (16 * t + n) * kRowPad + 16 * g;
      sc[t] = mfma_16x16x32<DT>(*reinterpret_cast<const uint4*>(row), qf[0], f32x4{0.f, 0.f, 0.f, 0.f});
      sc[t] = mfma_16x16x32<DT>(*reinterpret_cast<const uint4*>(row + 64), qf[1], sc[t]);
    }
    // V^T operands of the 4 dim blocks, transposed by the loads themselves.
    uint4 vt[4];
    {
      const char* row_a = lds_v + vt_key * kRowPad + vt_col;
      const char* row_b = row_a + 16 * kRowPad;
#pragma unroll
      for (int db = 0; db < 4; ++db) vt[db] = vt_operand(row_a, row_b, db);
    }
    __builtin_amdgcn_wave_barrier();
    // Scores of keys base + 16t + 4g + i for query n, masked past the chunk's end.
    float sv[8];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) sv[4 * t + i] = sc[t][i] * p.scale_log2;
    if (base + STEP > t_end || (PAGED && mask != 0xffffffffu)) {  // wave-uniform: a chunk's last step or an invalid block
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int kk = 16 * t + 4 * g + i;
          const bool ok = base + kk < t_end && (!PAGED || ((mask >> kk) & 1u));
          sv[4 * t + i] = ok ? sv[4 * t + i] : kNegInf;
        }
    }
    float mx = kNegInf;
#pragma unroll
    for (int i = 0; i < 8; ++i) mx = max_score(mx, sv[i]);
    // Lazy rescaling (kLazyMaxLog2). A lane's own 8 keys decide whether the reference moves;
    // only then is the maximum taken over the query's 4 lane groups (a permlane swap of a
    // register with itself leaves a lane's own value in one result, its partner's in the other).
    if (__builtin_amdgcn_ballot_w64(mx > m + kLazyMaxLog2) != 0) {  // wave-uniform
      const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
      mx = max_score(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
      const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
      mx = max_score(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
      const float mn = max_score(m, mx);
      ref = mn == kNegInf ? 0.f : mn;
      const float alpha = __builtin_amdgcn_exp2f(m - ref);
#pragma unroll
      for (int db = 0; db < 4; ++db) acc[db] *= alpha;
      l *= alpha;
      m = mn;
    }
    // P^T operand. fp16 rounds P once (unit roundoff 2^-11) and the row sums add the rounded
    // values; bf16 (2^-8) splits P into a rounded head and the rounded remainder, two products
    // with the same V^T, so the weights keep ~16 bits and the sums use P itself.
    uint32_t pw[4], pr[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float p0 = __builtin_amdgcn_exp2f(sv[2 * k] - ref);
      const float p1 = __builtin_amdgcn_exp2f(sv[2 * k + 1] - ref);
      const uint32_t w = pack2<DT>(p0, p1);
      pw[k] = w;
      if constexpr (DT == SKV_BF16) {
        pr[k] = pack2<DT>(p0 - lo16<DT>(w), p1 - hi16<DT>(w));
        l += p0 + p1;
      } else {
        l += lo16<DT>(w) + hi16<DT>(w);
      }
    }
    const uint4 pt = make_uint4(pw[0], pw[1], pw[2], pw[3]);
    const uint4 prt = make_uint4(pr[0], pr[1], pr[2], pr[3]);
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      acc[db] = mfma_16x16x32<DT>(vt[db], pt, acc[db]);
      if constexpr (DT == SKV_BF16) acc[db] = mfma_16x16x32<DT>(vt[db], prt, acc[db]);
    }
  };
  // Software pipeline: the next step's loads are in flight while this step computes.
  const int stride = kWaves * STEP;
  int s0 = t_begin + wave * STEP;
  uint4 ka[4], va[4], kb2[4], vb2[4];
  uint32_t ma = 0u, mb = 0u;
  if (s0 < t_end) ma = load_step(s0, ka, va);
  while (s0 < t_end) {
    const int s1 = s0 + stride;
    if (s1 < t_end) mb = load_step(s1, kb2, vb2);
    __builtin_amdgcn_sched_barrier(0);
    compute_step(s0, ka, va, ma);
    if (s1 >= t_end) break;
    const int s2 = s1 + stride;
    if (s2 < t_end) ma = load_step(s2, ka, va);
    __builtin_amdgcn_sched_barrier(0);
    compute_step(s1, kb2, vb2, mb);
    s0 = s2;
  }
  // Row sums over the 4 lane groups (the max is already common to them).
  l += xor_lane<16>(l);
  l += xor_lane<32>(l);

  // Merge the waves: wave w then finalises dim block w for the 16 queries. The merge buffer
  // overlaps the other waves' staging rows, so every wave leaves its key loop first.
  __syncthreads();
  if (g == 0) {
    s_m[wave][n] = m;
    s_l[wave][n] = l;
  }
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int i = 0; i < 4; ++i) s_acc[wave][n][16 * db + 4 * g + i] = acc[db][i];
  __syncthreads();
  if (wave >= 4) return;
  float M = kNegInf;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_m[w][n]);
  const float mref = M == kNegInf ? 0.f : M;
  float L = 0.f, A[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const float e = __builtin_amdgcn_exp2f(s_m[w][n] - mref);
    L += e * s_l[w][n];
#pragma unroll
    for (int i = 0; i < 4; ++i) A[i] += e * s_acc[w][n][16 * wave + 4 * g + i];
  }
  if (!q_ok) return;
  const int d0 = 16 * wave + 4 * g;
  if (nchunks == 1) {
    const float inv = L > 0.f ? 1.f / L : 0.f;
    uint2* o = reinterpret_cast<uint2*>(p.o + (int64_t)b * p.osb + (int64_t)qi * p.osq + (int64_t)h * p.osh);
    o[d0 / 4] = make_uint2(pack2<DT>(A[0] * inv, A[1] * inv), pack2<DT>(A[2] * inv, A[3] * inv));
    return;
  }
  const int64_t rh = ((int64_t)b * p.qlen + qi) * p.heads + h;
  float* rec = p.part + (rh * p.nchunk_max + chunk) * PSTRIDE;
  *reinterpret_cast<float4*>(rec + kPartPad + d0) = make_float4(A[0], A[1], A[2], A[3]);
  if (wave == 0 && g == 0) *reinterpret_cast<float2*>(rec) = make_float2(M, L);
}

// ---------------------------------------------------------------------------
// Multi-query attention with many queries per row (encoder attention over a
// table of encoder blocks, q_len = T; long prompts), fp16/bf16, head_dim 64,
// non-causal: one workgroup owns 64 queries of one (row, head), 16 per wave, and
// walks the row's keys in 64-key steps staged in LDS, so K/V are read once per
// 64 queries (mq_attention_kernel reads them once per 16). The workgroup is two
// parts of 4 waves: part 0 takes the first half of the steps, part 1 the second,
// each wave keeping its 16 queries' softmax state over its part's keys, and part 1
// hands its state to part 0 through LDS at the end. The split puts 4 waves on each
// SIMD (at most 128 VGPRs each) where one part alone would leave 2: the per-step chain
// (products, softmax, products) is latency-bound, not issue-bound. Each wave runs
// the same products as mq_attention_kernel on each 32-key half of the shared step; both
// halves' score products issue before the first half's softmax, so they overlap it.
// Steps are double-buffered in LDS (80 KB per workgroup) with one barrier per step
// that orders LDS only; every wave keeps the next step's global loads in flight (16
// key rows of K and of V, 8 lanes per 128-byte row) and reads their block ids with
// scalar loads when it issues them.
// ---------------------------------------------------------------------------
constexpr int kMqtQueries = 64;  // queries per workgroup, 16 per wave of a part
constexpr int kMqtParts = 2;     // key halves per workgroup

template <int DT, bool PAGED>
__global__ __launch_bounds__(64 * kWaves * kMqtParts) __attribute__((amdgpu_waves_per_eu(4))) void
mqt_attention_kernel(AttnParams p) {
  static_assert(kWaves * kMqQueries == kMqtQueries, "mqt_attention_kernel: 16 queries per wave");
  static_assert(kMqtParts == 2, "mqt_attention_kernel: the end-of-kernel merge is written for two parts");
  constexpr int D = 64;
  constexpr int STEP = 32;                       // keys per compute half-step
  constexpr int LSTEP = 64;                      // keys per staged step, 16 per wave
  constexpr int kRowPad = D * 2 + 32;            // LDS row of one key: 128 bytes + 32 of padding
  constexpr int kTileBytes = 2 * LSTEP * kRowPad; // K rows, then V rows
  __shared__ __attribute__((aligned(16))) char s_tiles[kMqtParts][2][kTileBytes];

  const int lane = threadIdx.x & 63;
  const int wave_all = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));  // wave-uniform
  const int wave = wave_all & (kWaves - 1);  // query tile
  const int part = wave_all / kWaves;        // key half
  char(*s_tile)[kTileBytes] = s_tiles[part];
  const int g = lane >> 4;  // lane group of the MFMA layouts
  const int n = lane & 15;  // query column (result, P^T) / key or dim row (operands)
  const int h = (int)(blockIdx.x % (uint32_t)p.heads);
  const int qg = (int)(blockIdx.x / (uint32_t)p.heads);
  const int b = blockIdx.y;
  const int kvh = p.group == 1 ? h : h / p.group;

  int len = p.lens[b];
  len = len < 0 ? 0 : (len > p.max_len ? p.max_len : len);
  const int qi = qg * kMqtQueries + wave * kMqQueries + n;  // this lane's query (result layout)
  const bool q_ok = qi < p.qlen;
  if (len == 0) {  // uniform over the workgroup: zero output
    if (q_ok && part == 0) {
      uint2* o = reinterpret_cast<uint2*>(p.o + (int64_t)b * p.osb + (int64_t)qi * p.osq + (int64_t)h * p.osh);
#pragma unroll
      for (int db = 0; db < 4; ++db) o[(16 * db + 4 * g) / 4] = make_uint2(0u, 0u);
    }
    return;
  }

  // Q^T operand: lane (query n, group g) holds dims 32s + 8g .. +8 for slabs s = 0, 1.
  uint4 qf[2];
#pragma unroll
  for (int sl = 0; sl < 2; ++sl) {
    qf[sl] = make_uint4(0u, 0u, 0u, 0u);
    if (q_ok) qf[sl] = p.q[(int64_t)b * p.qsb + (int64_t)qi * p.qsq + (int64_t)h * p.qsh + sl * 4 + g];
  }

  // Descriptors over the row's (slot, head) span (contiguous) or over the whole pool (paged).
  const char* kb = reinterpret_cast<const char*>(p.k);
  const char* vb = reinterpret_cast<const char*>(p.v);
  uint32_t row_bytes, col_base = 0;
  const uint32_t* trow = nullptr;
  if constexpr (PAGED) {
    row_bytes = (uint32_t)p.row_vecs * 16u;
    col_base = (uint32_t)kvh * (uint32_t)(D * 2);
    trow = reinterpret_cast<const uint32_t*>(p.tables + (int64_t)(p.trows ? p.trows[b] : b) * p.tstride);
  } else {
    const int slot = p.slots ? p.slots[b] : b;
    kb += ((int64_t)slot * p.ss + (int64_t)kvh * p.sh) * 16;
    vb += ((int64_t)slot * p.ss + (int64_t)kvh * p.sh) * 16;
    row_bytes = (uint32_t)p.st * 16u;
  }
  const __amdgpu_buffer_rsrc_t kres =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(kb), (short)0, (int)p.kv_bytes, kBufWord3);
  const __amdgpu_buffer_rsrc_t vres =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(vb), (short)0, (int)p.kv_bytes, kBufWord3);

  // Whether every block id under [0, len) is a pool block (the normal case): one vector
  // read of the table row; the steps' presence bits then depend on len only.
  bool row_ok = true;
  if constexpr (PAGED) {
    const int nblk = (len + p.bs - 1) >> p.bs_shift;
    bool bad = false;
    for (int e = lane; e < nblk; e += 64) bad |= trow[e] >= (uint32_t)p.nb;
    row_ok = __builtin_amdgcn_ballot_w64(bad) == 0;
  }

  // This part's steps: [st0, st0 + nsteps) of the row's ceil(len / 64), keys below lim.
  const int nsteps = ((len + LSTEP - 1) / LSTEP + kMqtParts - 1) / kMqtParts;
  const int st0 = part * nsteps;
  const int lim = min(len, (st0 + nsteps) * LSTEP);

  // Issues step st's loads for this wave (keys st*64 + 16*wave + 8r + (lane >> 3) for
  // r = 0, 1, byte column 16 * (lane & 7); at or past lim, or behind an invalid block,
  // the offset is out of range and the load returns zeros without a memory access) and
  // returns the step's presence bits: bit j for key st*64 + j in the softmax
  // (wave-uniform). Block ids are read with scalar loads (one per 8 keys, block size
  // >= 8, clamped to the row's last key so the index stays inside the row): the
  // wave's own two, and on a row with an invalid id the step's eight, in one batch.
  const int nat_row = lane >> 3, nat_col = (lane & 7) * 16;
  auto issue = [&](int st, uint4 (&kr)[2], uint4 (&vr)[2]) -> uint64_t {
    const int base = st * LSTEP;
    uint64_t bits = base + LSTEP <= len ? ~0ull : (base < len ? (1ull << (len - base)) - 1ull : 0ull);
    if constexpr (PAGED) {
      if (!row_ok) {
        uint32_t blk[8];
#pragma unroll
        for (int gi = 0; gi < 8; ++gi) blk[gi] = trow[(uint32_t)min(base + 8 * gi, len - 1) >> p.bs_shift];
#pragma unroll
        for (int gi = 0; gi < 8; ++gi)
          if (blk[gi] >= (uint32_t)p.nb) bits &= ~(0xffull << (8 * gi));
      }
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int key0 = base + 16 * wave + 8 * r;
      const int key = key0 + nat_row;
      uint32_t off;
      if constexpr (PAGED) {
        const uint32_t own = trow[(uint32_t)min(key0, len - 1) >> p.bs_shift];
        off = key < lim && own < (uint32_t)p.nb
                  ? (own * (uint32_t)p.bs + ((uint32_t)key & ((uint32_t)p.bs - 1u))) * row_bytes + col_base +
                        (uint32_t)nat_col
                  : kBufOutOfRange;
      } else {
        off = key < lim ? (uint32_t)key * row_bytes + (uint32_t)nat_col : kBufOutOfRange;
      }
      kr[r] = load_buf(kres, off);
      vr[r] = load_buf(vres, off);
    }
    return bits;
  };
  auto stage = [&](int buf, const uint4 (&kr)[2], const uint4 (&vr)[2]) {
    char* t = s_tile[buf];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int row = 16 * wave + 8 * r + nat_row;
      *reinterpret_cast<uint4*>(t + row * kRowPad + nat_col) = kr[r];
      *reinterpret_cast<uint4*>(t + LSTEP * kRowPad + row * kRowPad + nat_col) = vr[r];
    }
  };

  // V^T operand chunks (vt_operand): lane 4kk + q of group g reads keys K_g[kk] and
  // K_g[4 + kk], dims 16 db + 4q .. +3.
  const int vt_key = 4 * g + ((lane & 15) >> 2);
  const int vt_col = 8 * (lane & 3);

  float m = kNegInf, l = 0.f;  // query n's state (m in units of scale * log2 e); l sums this lane group's keys
  float ref = 0.f;             // m, or 0 while m is -inf: the exponents' offset
  f32x4 acc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  // fp16 sums P on the matrix cores: a product with an operand of ones gives every lane
  // its query's sum over the step's 32 keys (the rounded weights, as the PV product
  // uses them). bf16 sums the unrounded weights on the VALU: its P is two operands.
  constexpr bool kOnesSum = DT == SKV_F16;
  f32x4 l4 = f32x4{0.f, 0.f, 0.f, 0.f};
  const uint4 ones = make_uint4(0x3c003c00u, 0x3c003c00u, 0x3c003c00u, 0x3c003c00u);

  // Scores of one 32-key half of the staged step (K operand of tile t, slab s: key 16t + n,
  // dims 32s + 8g .. +8).
  auto scores = [&](int buf, int half, f32x4 (&sc)[2]) __attribute__((always_inline)) {
    const char* lds_k = s_tile[buf] + half * STEP * kRowPad;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const char* row = lds_k + (16 * t + n) * kRowPad + 16 * g;
      sc[t] = mfma_16x16x32<DT>(*reinterpret_cast<const uint4*>(row), qf[0], f32x4{0.f, 0.f, 0.f, 0.f});
      sc[t] = mfma_16x16x32<DT>(*reinterpret_cast<const uint4*>(row + 64), qf[1], sc[t]);
    }
  };
  // Softmax and PV products of one half; keys whose bit is clear score -inf.
  auto compute = [&](int buf, int half, const f32x4 (&sc)[2], uint32_t bits) __attribute__((always_inline)) {
    const char* lds_v = s_tile[buf] + LSTEP * kRowPad + half * STEP * kRowPad;
    uint4 vt[4];
    {
      const char* row_a = lds_v + vt_key * kRowPad + vt_col;
      const char* row_b = row_a + 16 * kRowPad;
#pragma unroll
      for (int db = 0; db < 4; ++db) vt[db] = vt_operand(row_a, row_b, db);
    }
    // Raw scores of keys 16t + 4g + i for query n. The scale (positive) multiplies
    // inside the exponent's FMA, so the maximum is taken on raw scores and scaled once.
    float sv[8];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) sv[4 * t + i] = sc[t][i];
    if (bits != 0xffffffffu) {  // wave-uniform: a row's last step or an invalid block
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          sv[4 * t + i] = ((bits >> (16 * t + 4 * g + i)) & 1u) ? sv[4 * t + i] : kNegInf;
    }
    float mx = kNegInf;
#pragma unroll
    for (int i = 0; i < 8; ++i) mx = max_score(mx, sv[i]);
    // Lazy rescaling (kLazyMaxLog2). A lane's own 8 keys decide whether the reference moves;
    // only then is the maximum taken over the query's 4 lane groups (a permlane swap of a
    // register with itself leaves a lane's own value in one result, its partner's in the other).
    if (__builtin_amdgcn_ballot_w64(mx * p.scale_log2 > m + kLazyMaxLog2) != 0) {  // wave-uniform
      const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
      mx = max_score(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
      const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
      mx = max_score(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
      const float mn = max_score(m, mx * p.scale_log2);
      ref = mn == kNegInf ? 0.f : mn;
      const float alpha = __builtin_amdgcn_exp2f(m - ref);
#pragma unroll
      for (int db = 0; db < 4; ++db) acc[db] *= alpha;
      if constexpr (kOnesSum)
        l4 *= alpha;
      else
        l *= alpha;
      m = mn;
    }
    // P^T operand, as in mq_attention_kernel: fp16 rounds P once and sums the rounded
    // values; bf16 adds the product of the rounded remainder.
    uint32_t pw[4], pr[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float p0 = __builtin_amdgcn_exp2f(fmaf(sv[2 * k], p.scale_log2, -ref));
      const float p1 = __builtin_amdgcn_exp2f(fmaf(sv[2 * k + 1], p.scale_log2, -ref));
      const uint32_t w = pack2<DT>(p0, p1);
      pw[k] = w;
      if constexpr (DT == SKV_BF16) {
        pr[k] = pack2<DT>(p0 - lo16<DT>(w), p1 - hi16<DT>(w));
        l += p0 + p1;
      }
    }
    const uint4 pt = make_uint4(pw[0], pw[1], pw[2], pw[3]);
    const uint4 prt = make_uint4(pr[0], pr[1], pr[2], pr[3]);
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      acc[db] = mfma_16x16x32<DT>(vt[db], pt, acc[db]);
      if constexpr (DT == SKV_BF16) acc[db] = mfma_16x16x32<DT>(vt[db], prt, acc[db]);
    }
    if constexpr (kOnesSum) l4 = mfma_16x16x32<DT>(ones, pt, l4);
  };

  // Step st's loads live in register slot st % 2 from their issue (one step ahead)
  // until they are staged into LDS buffer st % 2 during step st - 1; its presence bits
  // ride along in pbits. The loop is unrolled by 2 so the slot indices are constants,
  // and loads are issued unconditionally (past the part's last step they are out of
  // range and return zeros without a memory access), so the wait before staging a step
  // counts only that step's loads. Both parts run the same number of steps, so every
  // wave reaches every barrier.
  uint4 kr[2][2], vr[2][2];
  uint64_t pbits[2];
  pbits[0] = issue(st0, kr[0], vr[0]);
  pbits[1] = issue(st0 + 1, kr[1], vr[1]);
  stage(0, kr[0], vr[0]);
  lds_barrier();
  auto body = [&](int st, auto slot_c) __attribute__((always_inline)) {
    constexpr int SLOT = decltype(slot_c)::value;  // st % 2
    const uint64_t bits = pbits[SLOT];
    if (st + 1 < nsteps) stage((st + 1) & 1, kr[SLOT ^ 1], vr[SLOT ^ 1]);
    pbits[SLOT] = issue(st0 + st + 2, kr[SLOT], vr[SLOT]);
    f32x4 sc0[2], sc1[2];
    scores(st & 1, 0, sc0);
    scores(st & 1, 1, sc1);  // issued before the first half's softmax, so the two overlap
    compute(st & 1, 0, sc0, (uint32_t)bits);
    compute(st & 1, 1, sc1, (uint32_t)(bits >> 32));  // a half with no key changes nothing
    lds_barrier();
  };
  for (int st = 0; st < nsteps; st += 2) {
    body(st, std::integral_constant<int, 0>{});
    if (st + 1 >= nsteps) break;
    body(st + 1, std::integral_constant<int, 1>{});
  }
  if constexpr (kOnesSum) {
    l = l4[0];
  } else {  // row sums over the 4 lane groups (the max is common to them)
    l += xor_lane<16>(l);
    l += xor_lane<32>(l);
  }
  // Part 1 hands (max, sum, accumulators) to part 0 through LDS: 18 floats per lane, one
  // block of 64 x 18 per query tile, in the tiles, which are free after the loop's last
  // barrier.
  float* xs = reinterpret_cast<float*>(&s_tiles[0][0][0]) + wave * (18 * 64);
  static_assert(kWaves * 18 * 64 * sizeof(float) <= sizeof(s_tiles), "mqt_attention_kernel: merge area");
  if (part == 1) {
    xs[lane] = m;
    xs[64 + lane] = l;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) xs[128 + (4 * db + i) * 64 + lane] = acc[db][i];
  }
  lds_barrier();
  if (part == 1 || !q_ok) return;
  {
    const float m1 = xs[lane], l1 = xs[64 + lane];
    const float mm = fmaxf(m, m1);
    const float ref = mm == kNegInf ? 0.f : mm;
    const float a0 = __builtin_amdgcn_exp2f(m - ref), a1 = __builtin_amdgcn_exp2f(m1 - ref);
    l = a0 * l + a1 * l1;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[db][i] = a0 * acc[db][i] + a1 * xs[128 + (4 * db + i) * 64 + lane];
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  uint2* o = reinterpret_cast<uint2*>(p.o + (int64_t)b * p.osb + (int64_t)qi * p.osq + (int64_t)h * p.osh);
#pragma unroll
  for (int db = 0; db < 4; ++db)
    o[(16 * db + 4 * g) / 4] =
        make_uint2(pack2<DT>(acc[db][0] * inv, acc[db][1] * inv), pack2<DT>(acc[db][2] * inv, acc[db][3] * inv));
}

// ---------------------------------------------------------------------------
// Host helpers.
// ---------------------------------------------------------------------------
int64_t workspace_bytes(int64_t rows, int64_t heads, int64_t d, int64_t nchunk_max) {
  if (nchunk_max <= 1) return 0;
  return rows * heads * nchunk_max * (d + kPartPad) * (int64_t)sizeof(float);
}

// Keys one wave covers per sub-chunk over contiguous K/V for (dtype, head_dim); 0 if
// unsupported. Chunks are multiples of it, hence of the paged kernel's shorter trip too.
int sub_tokens(int32_t dtype, int32_t d) {
  const int eb = elt_bytes(dtype);
  if (eb == 0 || d <= 0) return 0;
  const int epl = 16 / eb;
  const int lpt = d / epl;
  if (lpt <= 0) return 0;
  const int tpi = 64 / lpt;
  int u = SKV_ATTN_SUB / tpi;
  u = u < 1 ? 1 : (u > SKV_ATTN_UNROLL ? SKV_ATTN_UNROLL : u);
  return tpi * u;
}

// cap_tokens > 0 bounds the chunk (rounded down to a whole sub-chunk): the general paged
// path stages a chunk's block ids in kMaxChunkBlocks LDS slots.
int32_t pick_chunk(int32_t rows, int32_t heads, int32_t d, int32_t max_len, int32_t dtype, int32_t cap_tokens = 0) {
  int sub = sub_tokens(dtype, d);
  if (sub <= 0) sub = 64;
  // A chunk is a whole number of workgroup passes (kWaves sub-chunks). Keep one chunk per
  // (row, head) — no partials, no merge launch — when there are (row, head) pairs to give
  // every CU ~4 workgroups, when a (row, head) holds at most 128 KB of K and V (its
  // workgroup streams that in less than the merge launch costs), or when there are 128+
  // pairs holding at most 512 KB each. Otherwise split the keys just enough to reach ~4
  // workgroups per CU. Measured (bf16, 20 heads x 64, graph-timed): paged ctx U[1, 452]
  // at batch 8 / 32: 9.25 -> 6.85 / 13.48 -> 9.31 us with one chunk; cross-attention over
  // 1500 keys at batch 8 / 48: 15.7 -> 13.7 / 61.3 -> 56.0 us; the split stays faster for
  // 1500 keys at batch 1-4 (8.1 vs 10.6 us at batch 1) and for 4096 keys at batch 8
  // (25.2 vs 35.9 us).
  const int64_t base = (int64_t)kWaves * sub;
  const int64_t target_wg = 1024;
  const int64_t rh = (int64_t)rows * heads;
  const int64_t max_chunks = cdiv(max_len > 0 ? max_len : 1, base);
  const int64_t item_bytes = (int64_t)(max_len > 0 ? max_len : 1) * 2 * d * elt_bytes(dtype);
  const bool one = rh >= target_wg || item_bytes <= ((int64_t)128 << 10) ||
                   (rh >= 128 && item_bytes <= ((int64_t)512 << 10));
  int64_t nchunks = one ? 1 : cdiv(target_wg, rh > 0 ? rh : 1);
  nchunks = nchunks < 1 ? 1 : (nchunks > max_chunks ? max_chunks : nchunks);
  const int64_t per = cdiv(max_len > 0 ? max_len : 1, nchunks);
  int64_t chunk = cdiv(per, base) * base;
  if (chunk > 16384) chunk = 16384;
  if (cap_tokens > 0 && chunk > cap_tokens) chunk = cap_tokens >= sub ? (cap_tokens / sub) * sub : sub;
  return (int32_t)chunk;
}

// Whether a paged call takes the fast path of attention_kernel: the pools fit the 32-bit
// buffer range and the block size is a power of two of at least the keys one load
// instruction of a wave covers (64 * elements per 16 bytes / head_dim).
bool paged_fast(int32_t dtype, int32_t d, int32_t kv_heads, int32_t bs, int32_t nb) {
  const int eb = elt_bytes(dtype);
  if (eb == 0 || d <= 0 || bs <= 0 || nb < 0) return false;
  const int epl = 16 / eb;
  const int64_t kv_bytes = (int64_t)nb * bs * ((int64_t)kv_heads * d / epl) * 16;
  return kv_bytes <= kBufLimit && (bs & (bs - 1)) == 0 && bs >= 64 * epl / d;
}

// Default chunk of a paged call: the general path keeps each chunk within
// kMaxChunkBlocks - 2 blocks (a chunk that starts mid-block spans one more).
int32_t paged_chunk(int32_t rows, int32_t heads, int32_t kv_heads, int32_t d, int32_t max_len, int32_t dtype,
                    int32_t bs, int32_t nb) {
  const int32_t cap = paged_fast(dtype, d, kv_heads, bs, nb) ? 0 : (kMaxChunkBlocks - 2) * bs;
  return pick_chunk(rows, heads, d, max_len, dtype, cap);
}

bool supported_d(int32_t d) { return d == 16 || d == 32 || d == 64 || d == 128; }

// Compute units of the current device (0 when the query fails), cached per device.
int device_cu_count() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cache[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (dev < kMaxDevices) {
    const int c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) n = 0;
  if (dev < kMaxDevices && n > 0) cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

template <int DT, int D, bool PAGED>
void launch_attention(const AttnParams& p, hipStream_t stream) {
  const int64_t rh = (int64_t)p.batch * p.qlen * p.heads;
  const dim3 grid = p.grid3d ? dim3((uint32_t)p.heads, (uint32_t)(p.batch * p.qlen), (uint32_t)p.nchunk_max)
                             : dim3((uint32_t)rh, (uint32_t)p.nchunk_max);
  constexpr int kTpi = 64 / (D / Elt<DT>::EPL);  // keys per load instruction of a wave
  const bool fast = p.kv_bytes <= kBufLimit && (!PAGED || (p.bs_shift >= 0 && (1 << p.bs_shift) >= kTpi));
  const uint32_t qlen_group = (uint32_t)p.qlen | ((uint32_t)p.group << 16);
  const uint32_t flags = (p.grid3d ? 1u : 0u) | (p.snake ? 2u : 0u) | (p.causal ? 4u : 0u) |
                         (PAGED && p.rank ? 8u : 0u) | ((uint32_t)p.cu_shift << 8) |
                         ((uint32_t)(p.bs_shift & 0xff) << 16);
  if (fast) {
    hipLaunchKernelGGL((attention_kernel<DT, D, PAGED, true>), grid, dim3(64 * kWaves), 0, stream, p.tables, p.lens,
                       p.trows, p.heads, p.tstride, p.max_len, p.chunk, qlen_group, flags, p.items, p.heads_magic, p);
  } else {
    hipLaunchKernelGGL((attention_kernel<DT, D, PAGED, false>), grid, dim3(64 * kWaves), 0, stream, p.tables, p.lens,
                       p.trows, p.heads, p.tstride, p.max_len, p.chunk, qlen_group, flags, p.items, p.heads_magic, p);
  }
  if (p.nchunk_max > 1)
    hipLaunchKernelGGL((merge_kernel<DT, D>), dim3((uint32_t)cdiv(rh, 4)), dim3(256), 0, stream, p);
}

template <bool PAGED>
int dispatch_attention(int32_t dtype, int32_t d, const AttnParams& p, hipStream_t stream) {
#define SKV_CASE(DT, DD)                        \
  if (dtype == DT && d == DD) {                 \
    launch_attention<DT, DD, PAGED>(p, stream); \
    return SKV_OK;                              \
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
                      int32_t d, int32_t max_len, float scale, int32_t causal, int32_t dtype, int32_t chunk) {
  const int eb = elt_bytes(dtype);
  if (eb == 0) return fail(SKV_EDTYPE, "%s: unknown dtype %d", who, dtype);
  if (!supported_d(d)) return fail(SKV_EINVAL, "%s: head_dim %d not in {16,32,64,128}", who, d);
  if (batch < 0 || q_len <= 0 || q_len > 65535 || heads <= 0 || heads > 65535 || kv_heads <= 0 ||
      heads % kv_heads != 0 || max_len < 0)
    return fail(SKV_EINVAL, "%s: bad sizes batch=%d q_len=%d (1..65535) heads=%d (1..65535) kv_heads=%d max_len=%d",
                who, batch, q_len, heads, kv_heads, max_len);
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
  // Grid: x = rows * heads workgroups (work-items must stay below 2^32), y = chunks.
  if ((int64_t)batch * q_len * heads * 64 * kWaves >= ((int64_t)1 << 32) || nchunk_max > 65535)
    return fail(SKV_EINVAL, "%s: launch too large (rows*heads=%lld, chunks=%d)", who,
                (long long)batch * q_len * heads, nchunk_max);
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
  p.grid3d = (int64_t)batch * q_len <= 65535;
  const int64_t items = (int64_t)batch * q_len * heads;
  const int cus = device_cu_count();
  p.snake = p.grid3d && nchunk_max == 1 && heads >= 2 && items * heads < ((int64_t)1 << 32) && cus > 0 &&
            (cus & (cus - 1)) == 0;
  if (p.snake) {
    p.cu_shift = __builtin_ctz((unsigned)cus);
    p.items = (uint32_t)items;
    p.heads_magic = (uint32_t)((((uint64_t)1 << 32) + (uint64_t)heads - 1) / (uint64_t)heads);
  }
  p.scale_log2 = scale * kLog2e;
  p.part = nullptr;
  return SKV_OK;
}

// The split-K partials of a launch whose rows span nchunk_max > 1 chunks go to the
// caller's workspace: check that it holds them and bind it.
int bind_workspace(AttnParams& p, const char* who, int32_t d, void* ws, int64_t ws_bytes) {
  const int64_t need = workspace_bytes((int64_t)p.batch * p.qlen, p.heads, d, p.nchunk_max);
  if (need > 0 && (!ws || ws_bytes < need || !aligned16(ws)))
    return fail(SKV_EWORKSPACE, "%s: workspace needs %lld bytes (16-byte aligned), got %lld", who, (long long)need,
                (long long)ws_bytes);
  p.part = need > 0 ? (float*)ws : nullptr;
  return SKV_OK;
}

}  // namespace

// The multi-query matrix-core attention (fp16/bf16, head_dim 64) and, for split rows, the merge.
template <bool PAGED>
void launch_mq(int32_t dtype, const AttnParams& p, hipStream_t s) {
  const int32_t qtiles = (int32_t)cdiv(p.qlen, kMqQueries);
  const dim3 grid((uint32_t)(p.heads * qtiles), (uint32_t)p.batch, (uint32_t)p.nchunk_max);
  if (dtype == SKV_BF16)
    hipLaunchKernelGGL((mq_attention_kernel<SKV_BF16, PAGED>), grid, dim3(64 * kWaves), 0, s, p, qtiles);
  else
    hipLaunchKernelGGL((mq_attention_kernel<SKV_F16, PAGED>), grid, dim3(64 * kWaves), 0, s, p, qtiles);
  if (p.nchunk_max > 1) {
    const int64_t rh = (int64_t)p.batch * p.qlen * p.heads;
    if (dtype == SKV_BF16)
      hipLaunchKernelGGL((merge_kernel<SKV_BF16, 64>), dim3((uint32_t)cdiv(rh, 4)), dim3(256), 0, s, p);
    else
      hipLaunchKernelGGL((merge_kernel<SKV_F16, 64>), dim3((uint32_t)cdiv(rh, 4)), dim3(256), 0, s, p);
  }
}

// Many queries per row on the matrix cores: 64 queries per workgroup over all of the row's keys.
template <bool PAGED>
void launch_mqt(int32_t dtype, const AttnParams& p, hipStream_t s) {
  const dim3 grid((uint32_t)(p.heads * cdiv(p.qlen, kMqtQueries)), (uint32_t)p.batch, 1u);
  if (dtype == SKV_BF16)
    hipLaunchKernelGGL((mqt_attention_kernel<SKV_BF16, PAGED>), grid, dim3(64 * kWaves * kMqtParts), 0, s, p);
  else
    hipLaunchKernelGGL((mqt_attention_kernel<SKV_F16, PAGED>), grid, dim3(64 * kWaves * kMqtParts), 0, s, p);
}

// Whether the 64-query kernel serves a multi-query launch: enough queries per row,
// (row, head, 64 queries) workgroups for at least three quarters of the compute units
// (it does not split keys across workgroups; below that the 16-query kernel, which
// does, is faster: encoder attention over 1500 bf16 positions, 6 heads (144
// workgroups) 20.4 vs 20.7 us, 8 heads (192) 23.2 vs 21.2 us, 20 heads over 750
// positions (240) 18.0 vs 13.4 us), and a positive scale (its maximum is taken on
// unscaled scores).
bool use_mqt(const AttnParams& p) {
  return p.qlen >= kMqtQueries && p.scale_log2 > 0.f &&
         4 * (int64_t)p.batch * p.heads * cdiv(p.qlen, kMqtQueries) >= 3 * (int64_t)device_cu_count() &&
         (int64_t)p.heads * cdiv(p.qlen, kMqtQueries) <= 0x7fffffff;
}

// ---------------------------------------------------------------------------
// Split-K scratch of skv_paged_attention_noalloc: a fixed device array, so that
// entry point allocates nothing. Each device holds its own copy for the life of
// the process; its address on the current device is looked up once per device
// (hipGetSymbolAddress) and kept. Host code never passes `scratch` itself to a
// kernel: on the host the name stands for a host-side shadow, not the device
// copy. Calls on one device share the array, so calls that overlap in time on
// one device (different streams) race on it.
// ---------------------------------------------------------------------------
constexpr int64_t kScratchBytes = (int64_t)4 << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxScratchDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxScratchDevices];
std::mutex g_scratch_mu;

// The current device's copy of `scratch` (looked up on the device's first call).
int scratch_on_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail((int)e, "scratch: hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(SKV_EINVAL, "scratch: device %d outside the %d devices the library tracks", dev, kMaxScratchDevices);
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p)
        return fail(e != hipSuccess ? (int)e : SKV_EINVAL, "scratch: hipGetSymbolAddress failed on device %d: %s", dev,
                    hipGetErrorString(e));
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return SKV_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI.
// ---------------------------------------------------------------------------
extern "C" {

// The build passes SKV_SOURCE_DIGEST: a hash of the sources, headers and code
// flags this library was compiled from, which the Python binding checks
// against the checked-out tree before it binds anything.
#ifndef SKV_SOURCE_DIGEST
#define SKV_SOURCE_DIGEST "unknown"
#endif
const char* skv_version(void) { return "speechkv 0.3.0 gfx950 src:" SKV_SOURCE_DIGEST; }

const char* skv_last_error(void) { return skv::last_error(); }

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
  if (total < ((int64_t)1 << 31)) {
    hipLaunchKernelGGL(append32_kernel, dim3((uint32_t)blocks, v_new ? 2 : 1), dim3(256), 0, (hipStream_t)stream,
                       (const uint4*)k_new, (const uint4*)(v_new ? v_new : k_new), new_stride_n / epl,
                       new_stride_h / epl, (uint4*)k_pool, (uint4*)(v_pool ? v_pool : k_pool), slot_mapping,
                       (uint32_t)total, make_div((uint32_t)(num_heads * vpr)), make_div((uint32_t)vpr), num_slots);
  } else {
    hipLaunchKernelGGL(append_kernel, dim3((uint32_t)blocks, v_new ? 2 : 1), dim3(256), 0, (hipStream_t)stream,
                       (const uint4*)k_new, (const uint4*)(v_new ? v_new : k_new), new_stride_n / epl,
                       new_stride_h / epl, (uint4*)k_pool, (uint4*)(v_pool ? v_pool : k_pool), slot_mapping,
                       n_tokens, num_heads, vpr, num_slots);
  }
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
  const bool pow2 = (block_size & (block_size - 1)) == 0 && (vpr & (vpr - 1)) == 0;
  const int64_t pool_bytes = (int64_t)num_blocks * block_size * num_heads * vpr * 16;
  if (pow2 && vpr <= 64 && 64 / vpr <= block_size && table_stride >= 1 && pool_bytes <= kBufLimit &&
      total < ((int64_t)1 << 31)) {
    const int64_t groups = cdiv(max_len, (int64_t)(64 / vpr) * kGatherLoads);
    const int64_t waves = (int64_t)batch * num_heads * groups;
    if (waves > 0 && cdiv(waves, 4) <= 0x7fffffff) {
      const DivU32 per_row = make_div((uint32_t)(num_heads * groups)), per_head = make_div((uint32_t)groups);
      hipLaunchKernelGGL(gather_rows_kernel, dim3((uint32_t)cdiv(waves, 4), v_pool ? 2 : 1), dim3(256), 0,
                         (hipStream_t)stream, (uint32_t)waves, per_row.d, per_row.m, per_head.d, per_head.m,
                         table_stride, __builtin_ctz((unsigned)block_size), __builtin_ctz((unsigned)vpr),
                         block_tables, lens, max_len, num_blocks, num_heads, (uint32_t)pool_bytes,
                         (const uint4*)k_pool, (const uint4*)(v_pool ? v_pool : k_pool), (uint4*)k_out,
                         (uint4*)(v_out ? v_out : k_out));
      return check_launch("skv_gather");
    }
  }
  if (total < ((int64_t)1 << 31)) {
    const uint32_t per_head = (uint32_t)cdiv(max_len, kGatherRows) * (uint32_t)vpr;
    const int64_t groups = (int64_t)batch * num_heads * per_head;
    int64_t gblocks = cdiv(groups, 256);
    if (gblocks > 65535) gblocks = 65535;
    hipLaunchKernelGGL(gather32_kernel, dim3((uint32_t)gblocks, v_pool ? 2 : 1), dim3(256), 0, (hipStream_t)stream,
                       (const uint4*)k_pool, (const uint4*)(v_pool ? v_pool : k_pool), block_tables, table_stride,
                       lens, (uint4*)k_out, (uint4*)(v_out ? v_out : k_out), (uint32_t)groups,
                       make_div(per_head * (uint32_t)num_heads), make_div(per_head), make_div((uint32_t)vpr),
                       make_div((uint32_t)block_size), num_heads, num_blocks, max_len);
  } else {
    hipLaunchKernelGGL(gather_kernel, dim3((uint32_t)blocks, v_pool ? 2 : 1), dim3(256), 0, (hipStream_t)stream,
                       (const uint4*)k_pool, (const uint4*)(v_pool ? v_pool : k_pool), block_tables, table_stride,
                       lens, (uint4*)k_out, (uint4*)(v_out ? v_out : k_out), batch, num_heads, vpr, block_size,
                       num_blocks, max_len);
  }
  return check_launch("skv_gather");
}

int skv_copy_cross_kv(const void* const* k_srcs, const void* const* v_srcs, int32_t n_layers, int64_t src_stride_h,
                      int64_t src_stride_t, void* dst, int64_t dst_stride_l, int64_t dst_stride_kv,
                      int64_t dst_stride_h, int64_t dst_stride_t, int32_t num_heads, int32_t n_tokens,
                      int32_t head_dim, int32_t dtype, void* stream) {
  const int eb = elt_bytes(dtype);
  if (eb == 0) return fail(SKV_EDTYPE, "skv_copy_cross_kv: unknown dtype %d", dtype);
  if (n_layers <= 0 || n_layers > kMaxCrossLayers || num_heads <= 0 || num_heads > 65535 || head_dim <= 0 ||
      n_tokens < 0)
    return fail(SKV_EINVAL, "skv_copy_cross_kv: bad sizes layers=%d (1..%d) heads=%d head_dim=%d n=%d", n_layers,
                kMaxCrossLayers, num_heads, head_dim, n_tokens);
  if (n_tokens == 0) return SKV_OK;
  if (!k_srcs || !v_srcs || !dst) return fail(SKV_EINVAL, "skv_copy_cross_kv: null pointer argument");
  const int epl = 16 / eb;
  const int vpr = head_dim / epl;
  if (head_dim % epl || (vpr & (vpr - 1)))
    return fail(SKV_EALIGN, "skv_copy_cross_kv: head_dim*%d bytes must be a power-of-two multiple of 16", eb);
  if (src_stride_h % epl || src_stride_t % epl || dst_stride_l % epl || dst_stride_kv % epl || dst_stride_h % epl ||
      dst_stride_t % epl)
    return fail(SKV_EALIGN, "skv_copy_cross_kv: strides must be multiples of %d elements", epl);
  CrossCopyParams p{};
  for (int l = 0; l < n_layers; ++l) {
    if (!k_srcs[l] || !v_srcs[l]) return fail(SKV_EINVAL, "skv_copy_cross_kv: null source for layer %d", l);
    if (!aligned16(k_srcs[l]) || !aligned16(v_srcs[l]))
      return fail(SKV_EALIGN, "skv_copy_cross_kv: sources must be 16-byte aligned");
    p.src[2 * l] = (const uint4*)k_srcs[l];
    p.src[2 * l + 1] = (const uint4*)v_srcs[l];
  }
  if (!aligned16(dst)) return fail(SKV_EALIGN, "skv_copy_cross_kv: destination must be 16-byte aligned");
  p.ssh = src_stride_h / epl;
  p.sst = src_stride_t / epl;
  p.dst = (uint4*)dst;
  p.dsl = dst_stride_l / epl;
  p.dskv = dst_stride_kv / epl;
  p.dsh = dst_stride_h / epl;
  p.dst_t = dst_stride_t / epl;
  p.n = n_tokens;
  p.vpr = vpr;
  p.vpr_shift = __builtin_ctz((unsigned)vpr);
  const int64_t per_head = (int64_t)n_tokens * vpr;
  int64_t bx = cdiv(per_head, 256 * kCopyVecs);
  if (bx > 65535) bx = 65535;
  hipLaunchKernelGGL(cross_copy_kernel, dim3((uint32_t)bx, (uint32_t)num_heads, (uint32_t)(2 * n_layers)), dim3(256),
                     0, (hipStream_t)stream, p);
  return check_launch("skv_copy_cross_kv");
}

int skv_argmax(const void* logits, int64_t row_stride, int32_t rows, int32_t vocab, int32_t dtype,
               int64_t* out_tokens, const int32_t* row_slots, int32_t num_slots, int64_t* slot_tokens,
               const int64_t* slot_eos, int32_t* slot_finished, int64_t* finished_count, void* stream) {
  const int eb = elt_bytes(dtype);
  if (eb == 0) return fail(SKV_EDTYPE, "skv_argmax: unknown dtype %d", dtype);
  if (rows < 0 || vocab <= 0 || vocab >= (1 << 29) || row_stride < vocab || num_slots < 0)
    return fail(SKV_EINVAL, "skv_argmax: bad sizes rows=%d vocab=%d row_stride=%lld num_slots=%d", rows, vocab,
                (long long)row_stride, num_slots);
  if (rows == 0) return SKV_OK;
  const bool eos = slot_eos || slot_finished || finished_count;
  if (!logits || !out_tokens || (eos && !(slot_eos && slot_finished && finished_count)) ||
      ((slot_tokens || eos) && !row_slots) || (row_slots && !slot_tokens && !eos))
    return fail(SKV_EINVAL, "skv_argmax: null pointer argument");
  SlotFeedback f{row_slots, num_slots, slot_tokens, slot_eos, slot_finished, (unsigned long long*)finished_count};
  const int64_t rb = row_stride * eb;
  // 16-byte vectors per thread for one pass over a row (its 32-bit words, rounded up).
  const int64_t per_thread = cdiv(cdiv((int64_t)vocab * eb, 16), kArgmaxThreads);
  const int vecs = per_thread <= 1 ? 1 : per_thread <= 2 ? 2 : per_thread <= 4 ? 4 : 7;
  switch (dtype) {
    case SKV_F32:
      launch_argmax<SKV_F32>(vecs, rows, (hipStream_t)stream, (const char*)logits, rb, vocab, out_tokens, f);
      break;
    case SKV_F16:
      launch_argmax<SKV_F16>(vecs, rows, (hipStream_t)stream, (const char*)logits, rb, vocab, out_tokens, f);
      break;
    default:
      launch_argmax<SKV_BF16>(vecs, rows, (hipStream_t)stream, (const char*)logits, rb, vocab, out_tokens, f);
      break;
  }
  return check_launch("skv_argmax");
}

int skv_add_layernorm(const void* x, int64_t ldx, const void* y, int64_t ldy, const void* gamma, const void* beta,
                      float eps, void* sum, int64_t lds, void* norm, int64_t ldn, int32_t rows, int32_t hidden,
                      int32_t dtype, void* stream) {
  const int eb = elt_bytes(dtype);
  if (eb == 0) return fail(SKV_EDTYPE, "skv_add_layernorm: unknown dtype %d", dtype);
  const int epl = 16 / eb;
  if (rows < 0 || hidden <= 0 || hidden % epl || hidden > 64 * 8 * epl)
    return fail(SKV_EINVAL, "skv_add_layernorm: hidden %d must be a multiple of %d and at most %d (rows=%d)", hidden,
                epl, 64 * 8 * epl, rows);
  if (rows == 0) return SKV_OK;
  if (!x || !gamma || !beta || !norm) return fail(SKV_EINVAL, "skv_add_layernorm: null pointer argument");
  if (!aligned16(x) || !aligned16(gamma) || !aligned16(beta) || !aligned16(norm) || (y && !aligned16(y)) ||
      (sum && !aligned16(sum)) || ldx % epl || ldy % epl || lds % epl || ldn % epl)
    return fail(SKV_EALIGN, "skv_add_layernorm: rows must be 16-byte aligned");
  if (!(eps >= 0.f)) return fail(SKV_EINVAL, "skv_add_layernorm: eps must be >= 0");
  AddNormParams p{};
  p.x = (const uint4*)x;
  p.y = (const uint4*)y;
  p.gamma = (const uint4*)gamma;
  p.beta = (const uint4*)beta;
  p.sum = y ? (uint4*)sum : nullptr;
  p.norm = (uint4*)norm;
  p.ldx = ldx / epl;
  p.ldy = ldy / epl;
  p.lds = lds / epl;
  p.ldn = ldn / epl;
  p.rows = rows;
  p.vecs = hidden / epl;
  p.eps = eps;
  p.inv_n = 1.f / (float)hidden;
  const int vpl = (int)cdiv(p.vecs, 64);
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case SKV_F32: launch_add_layernorm<SKV_F32>(p, vpl, s); break;
    case SKV_F16: launch_add_layernorm<SKV_F16>(p, vpl, s); break;
    default: launch_add_layernorm<SKV_BF16>(p, vpl, s); break;
  }
  return check_launch("skv_add_layernorm");
}

int skv_codebook_embed_sum(const int64_t* codes, int64_t codes_stride, int32_t rows, const void* const* tables,
                           int32_t num_codebooks, int32_t vocab, int32_t dim, void* out, int64_t out_stride,
                           int32_t dtype, void* stream) {
  const int eb = elt_bytes(dtype);
  if (eb == 0) return fail(SKV_EDTYPE, "skv_codebook_embed_sum: unknown dtype %d", dtype);
  const int epl = 16 / eb;
  if (rows < 0 || num_codebooks < 1 || num_codebooks > kMaxCodebooks || vocab <= 0 || dim <= 0 || dim % epl)
    return fail(SKV_EINVAL, "skv_codebook_embed_sum: bad sizes rows=%d codebooks=%d (1..%d) vocab=%d dim=%d "
                "(a multiple of %d)", rows, num_codebooks, kMaxCodebooks, vocab, dim, epl);
  if (rows == 0) return SKV_OK;
  if (!codes || !tables || !out) return fail(SKV_EINVAL, "skv_codebook_embed_sum: null pointer argument");
  if (codes_stride < num_codebooks || out_stride < dim || out_stride % epl || !aligned16(out))
    return fail(SKV_EALIGN, "skv_codebook_embed_sum: bad strides (codes %lld, out %lld) or unaligned output",
                (long long)codes_stride, (long long)out_stride);
  EmbedSumParams p{};
  for (int k = 0; k < num_codebooks; ++k) {
    if (!tables[k] || !aligned16(tables[k]))
      return fail(SKV_EALIGN, "skv_codebook_embed_sum: table %d is null or not 16-byte aligned", k);
    p.tables[k] = (const uint4*)tables[k];
  }
  p.codes = codes;
  p.codes_stride = codes_stride;
  p.out = (uint4*)out;
  p.out_stride = out_stride / epl;
  p.books = num_codebooks;
  p.vocab = vocab;
  p.vecs = dim / epl;
  p.total = (int64_t)rows * p.vecs;
  if (p.total >= ((int64_t)1 << 32) - 256)  // work-items of one launch stay below 2^32
    return fail(SKV_EINVAL, "skv_codebook_embed_sum: %d rows of %d vectors are too many", rows, p.vecs);
  const int64_t blocks = cdiv(p.total, 256);
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((uint32_t)blocks);
  switch (dtype) {
    case SKV_F32: hipLaunchKernelGGL(embed_sum_kernel<SKV_F32>, grid, dim3(256), 0, s, p); break;
    case SKV_F16: hipLaunchKernelGGL(embed_sum_kernel<SKV_F16>, grid, dim3(256), 0, s, p); break;
    default: hipLaunchKernelGGL(embed_sum_kernel<SKV_BF16>, grid, dim3(256), 0, s, p); break;
  }
  return check_launch("skv_codebook_embed_sum");
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

int32_t skv_paged_chunk_tokens(int32_t rows, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                               int32_t max_ctx, int32_t dtype, int32_t block_size, int32_t num_blocks) {
  return paged_chunk(rows, num_heads, num_kv_heads > 0 ? num_kv_heads : num_heads, head_dim, max_ctx, dtype,
                     block_size, num_blocks);
}

}  // extern "C"

namespace {

// skv_paged_attention with a workspace (the caller's, or the library's
// fixed scratch for the allocation-free entry point).
int paged_attention_impl(const char* who, const void* q, int64_t q_stride_b, int64_t q_stride_q, int64_t q_stride_h,
                         void* k_pool, void* v_pool, const int32_t* block_tables, int32_t table_stride,
                         const int32_t* table_rows, const int32_t* ctx_lens, const void* k_new, const void* v_new,
                         int64_t new_stride_b, int64_t new_stride_q, int64_t new_stride_h, void* out,
                         int64_t o_stride_b, int64_t o_stride_q, int64_t o_stride_h, int32_t batch, int32_t q_len,
                         int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                         int32_t num_blocks, int32_t max_ctx, float scale, int32_t causal, int32_t dtype,
                         int32_t chunk_tokens, void* workspace, int64_t ws_bytes, bool fixed_scratch,
                         void* stream) {
  // causal is a flags word: SKV_ATTN_CAUSAL, and SKV_ATTN_ROWS_LONGEST_FIRST when the caller's rows
  // already come longest-first (the launch then keeps their order instead of ranking them).
  const bool longest_first = (causal & SKV_ATTN_ROWS_LONGEST_FIRST) != 0;
  causal &= SKV_ATTN_CAUSAL;
  if (block_size < 2 || num_blocks < 0 || table_stride <= 0 || !block_tables)
    return fail(SKV_EINVAL, "%s: bad block table arguments (block_size must be >= 2)", who);
  if ((k_new == nullptr) != (v_new == nullptr))
    return fail(SKV_EINVAL, "%s: k_new and v_new must both be given or both be NULL", who);
  const int64_t table_cap = (int64_t)table_stride * block_size;
  if (max_ctx > table_cap) max_ctx = (int32_t)table_cap;
  // The general paged path (a block size that is not a power of two of at least one load
  // instruction's keys, or a pool past the 32-bit buffer range) stages a chunk's block ids in
  // kMaxChunkBlocks LDS slots, so its default chunk stays within that many blocks; the fast
  // path and the multi-query kernels read block ids with scalar loads and take chunks of any
  // length.
  const bool fast = elt_bytes(dtype) != 0 && paged_fast(dtype, head_dim, num_kv_heads, block_size, num_blocks);
  if (chunk_tokens <= 0 && elt_bytes(dtype) != 0 && num_kv_heads > 0 && supported_d(head_dim))
    chunk_tokens = paged_chunk(batch * q_len, num_heads, num_kv_heads, head_dim, max_ctx > 0 ? max_ctx : 1, dtype,
                               block_size, num_blocks);
  AttnParams p{};
  int rc = prepare_attention(p, who, q, q_stride_b, q_stride_q, q_stride_h, k_pool, v_pool, out, o_stride_b,
                             o_stride_q, o_stride_h, ctx_lens, batch, q_len, num_heads, num_kv_heads, head_dim,
                             max_ctx, scale, causal, dtype, chunk_tokens);
  if (rc != SKV_OK) return rc;
  if (!fast && p.chunk / block_size + 2 > kMaxChunkBlocks)
    return fail(SKV_EINVAL, "%s: chunk_tokens %d spans more than %d blocks of %d (pass a smaller chunk_tokens)", who,
                p.chunk, kMaxChunkBlocks - 2, block_size);
  if (k_new) {
    const int epl = 16 / elt_bytes(dtype);
    if (!aligned16(k_new) || !aligned16(v_new) || new_stride_b % epl || new_stride_q % epl || new_stride_h % epl)
      return fail(SKV_EALIGN, "%s: k_new/v_new must be 16-byte aligned with strides in %d-element units", who, epl);
    p.kn = (const uint4*)k_new;
    p.vn = (const uint4*)v_new;
    p.nsb = new_stride_b / epl;
    p.nsq = new_stride_q / epl;
    p.nsh = new_stride_h / epl;
  }
  p.tables = block_tables;
  p.tstride = table_stride;
  p.trows = table_rows;
  p.bs = block_size;
  p.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz((unsigned)block_size) : -1;
  p.nb = num_blocks;
  p.row_vecs = (int64_t)num_kv_heads * head_dim / (16 / elt_bytes(dtype));
  p.kv_bytes = (int64_t)num_blocks * block_size * p.row_vecs * 16;
  // Several non-causal queries per row with no fused append (attention over a whole encoder
  // table, EncoderAttentionBackend): every 16 queries of a row share one read of its blocks;
  // the 64-query kernel takes all of a row's keys in one workgroup, so it needs no partials.
  const bool mq = !p.causal && q_len >= 2 && !k_new && head_dim == 64 && (dtype == SKV_F16 || dtype == SKV_BF16) &&
                  p.kv_bytes <= kBufLimit && p.bs_shift >= 3 && batch <= 65535;
  const bool mqt = mq && use_mqt(p);
  if (mqt) {
    p.nchunk_max = 1;
    p.snake = 0;
  }
  p.rank = p.snake && q_len == 1 && batch <= kRankRows && !longest_first;
  rc = bind_workspace(p, who, head_dim, workspace, ws_bytes);
  if (rc != SKV_OK) {
    if (!fixed_scratch) return rc;
    return fail(SKV_EWORKSPACE,
                "%s: this call needs %lld bytes of split-K partials, more than the %lld bytes of the library's fixed "
                "scratch; use skv_paged_attention with a workspace, or larger chunk_tokens", who,
                (long long)workspace_bytes((int64_t)batch * q_len, num_heads, head_dim, p.nchunk_max),
                (long long)ws_bytes);
  }
  if (batch == 0) return SKV_OK;
  if (mq) {
    if (mqt)
      launch_mqt<true>(dtype, p, (hipStream_t)stream);
    else
      launch_mq<true>(dtype, p, (hipStream_t)stream);
    return check_launch(who);
  }
  rc = dispatch_attention<true>(dtype, head_dim, p, (hipStream_t)stream);
  if (rc != SKV_OK) return rc;
  return check_launch(who);
}

}  // namespace

extern "C" {

int skv_paged_attention(const void* q, int64_t q_stride_b, int64_t q_stride_q, int64_t q_stride_h,
                        void* k_pool, void* v_pool, const int32_t* block_tables, int32_t table_stride,
                        const int32_t* table_rows, const int32_t* ctx_lens, const void* k_new, const void* v_new,
                        int64_t new_stride_b, int64_t new_stride_q, int64_t new_stride_h, void* out,
                        int64_t o_stride_b, int64_t o_stride_q, int64_t o_stride_h, int32_t batch, int32_t q_len,
                        int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                        int32_t num_blocks, int32_t max_ctx, float scale, int32_t causal, int32_t dtype,
                        int32_t chunk_tokens, void* workspace, int64_t workspace_bytes, void* stream) {
  return paged_attention_impl("skv_paged_attention", q, q_stride_b, q_stride_q, q_stride_h, k_pool, v_pool,
                              block_tables, table_stride, table_rows, ctx_lens, k_new, v_new, new_stride_b,
                              new_stride_q, new_stride_h, out, o_stride_b, o_stride_q, o_stride_h, batch, q_len,
                              num_heads, num_kv_heads, head_dim, block_size, num_blocks, max_ctx, scale, causal,
                              dtype, chunk_tokens, workspace, workspace_bytes, false, stream);
}

int skv_paged_attention_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_q, int64_t q_stride_h,
                                void* k_pool, void* v_pool, const int32_t* block_tables, int32_t table_stride,
                                const int32_t* table_rows, const int32_t* ctx_lens, const void* k_new,
                                const void* v_new, int64_t new_stride_b, int64_t new_stride_q, int64_t new_stride_h,
                                void* out, int64_t o_stride_b, int64_t o_stride_q, int64_t o_stride_h, int32_t batch,
                                int32_t q_len, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                int32_t block_size, int32_t num_blocks, int32_t max_ctx, float scale, int32_t causal,
                                int32_t dtype, int32_t chunk_tokens, void* stream) {
  void* ws = nullptr;
  const int rc = scratch_on_current_device(&ws);
  if (rc != SKV_OK) return rc;
  return paged_attention_impl("skv_paged_attention_noalloc", q, q_stride_b, q_stride_q, q_stride_h, k_pool, v_pool,
                              block_tables, table_stride, table_rows, ctx_lens, k_new, v_new, new_stride_b,
                              new_stride_q, new_stride_h, out, o_stride_b, o_stride_q, o_stride_h, batch, q_len,
                              num_heads, num_kv_heads, head_dim, block_size, num_blocks, max_ctx, scale, causal,
                              dtype, chunk_tokens, ws, kScratchBytes, true, stream);
}

int skv_dense_attention(const void* q, int64_t q_stride_b, int64_t q_stride_q, int64_t q_stride_h, const void* k,
                        const void* v, int64_t kv_stride_s, int64_t kv_stride_h, int64_t kv_stride_t,
                        const int32_t* slot_ids, const int32_t* lens, void* out, int64_t o_stride_b,
                        int64_t o_stride_q, int64_t o_stride_h, int32_t batch, int32_t q_len, int32_t num_heads,
                        int32_t num_kv_heads, int32_t head_dim, int32_t max_len, float scale, int32_t causal,
                        int32_t dtype, int32_t chunk_tokens, void* workspace, int64_t workspace_bytes, void* stream) {
  AttnParams p{};
  int rc = prepare_attention(p, "skv_dense_attention", q, q_stride_b, q_stride_q, q_stride_h, k, v, out, o_stride_b,
                             o_stride_q, o_stride_h, lens, batch, q_len, num_heads, num_kv_heads, head_dim, max_len,
                             scale, causal, dtype, chunk_tokens);
  if (rc != SKV_OK) return rc;
  const int epl = 16 / elt_bytes(dtype);
  if (kv_stride_s % epl || kv_stride_h % epl || kv_stride_t % epl)
    return fail(SKV_EALIGN, "skv_dense_attention: K/V strides must be multiples of %d elements", epl);
  p.ss = kv_stride_s / epl;
  p.sh = kv_stride_h / epl;
  p.st = kv_stride_t / epl;
  // One (slot, head) span: max_len keys at the key stride, plus one key row.
  p.kv_bytes = max_len > 0 ? ((int64_t)(max_len - 1) * (p.st < 0 ? -p.st : p.st) + head_dim / epl) * 16 : 16;
  if (p.st < 0) p.kv_bytes = kBufLimit + 1;  // negative key strides take the 64-bit path
  p.slots = slot_ids;
  // Several non-causal queries per row (a prompt's cross-attention): one workgroup per
  // tile of 16 queries reads the row's K/V once and runs both products on the matrix cores;
  // the 64-query kernel takes all of a row's keys in one workgroup (no partials).
  const bool mq = !p.causal && q_len >= 2 && head_dim == 64 && (dtype == SKV_F16 || dtype == SKV_BF16) &&
                  p.kv_bytes <= kBufLimit && p.st > 0 && batch <= 65535;
  const bool mqt = mq && use_mqt(p);
  if (mqt) {
    p.nchunk_max = 1;
    p.snake = 0;
  }
  rc = bind_workspace(p, "skv_dense_attention", head_dim, workspace, workspace_bytes);
  if (rc != SKV_OK) return rc;
  if (batch == 0) return SKV_OK;
  if (mq) {
    if (mqt)
      launch_mqt<false>(dtype, p, (hipStream_t)stream);
    else
      launch_mq<false>(dtype, p, (hipStream_t)stream);
    return check_launch("skv_dense_attention");
  }
  rc = dispatch_attention<false>(dtype, head_dim, p, (hipStream_t)stream);
  if (rc != SKV_OK) return rc;
  return check_launch("skv_dense_attention");
}

}  // extern "C"
