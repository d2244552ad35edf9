// Device-side bookkeeping of one MTP cycle, so the whole cycle (draft k, verify
// k + 1, accept, commit) can be captured once in a HIP graph and replayed with a
// single host synchronisation. Every quantity that varies between cycles - the
// accepted count, the drawn token, the pending (hidden, token) pairs of the MTP
// head, the uniforms' draw counter - lives in device memory read by these kernels.
//
// Reference: the host-side bookkeeping of decode() (engine/speculative.py:82-102):
// mx.eval + accept.item(), pend_h / pend_ids, feed.
//
// Uniforms: Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC 2011), a counter-based
// generator, so a draw needs only (seed, draw counter) and the stream never
// repeats or runs out: draw event c gives
//   u(c, i) = (philox({c_lo, c_hi, i / 4, 0}, {seed_lo, seed_hi})[i % 4] >> 8) * 2^-24.
// The reference draws from MLX's generator (engine/speculative.py:79-81).
#include "qvex_common.h"

namespace {

__device__ __forceinline__ float philox_uniform(uint64_t seed, uint64_t event, int i) {
  uint32_t c0 = (uint32_t)event, c1 = (uint32_t)(event >> 32), c2 = (uint32_t)(i >> 2), c3 = 0u;
  uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r > 0) {
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    const uint32_t lo0 = 0xD2511F53u * c0, hi0 = __umulhi(0xD2511F53u, c0);
    const uint32_t lo1 = 0xCD9E8D57u * c2, hi1 = __umulhi(0xCD9E8D57u, c2);
    const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0;
    c1 = lo1;
    c2 = n2;
    c3 = lo0;
  }
  const int w = i & 3;
  const uint32_t x = w == 0 ? c0 : (w == 1 ? c1 : (w == 2 ? c2 : c3));
  return (float)(x >> 8) * 0x1p-24f;
}

// out[i] = u(*counter, i) for i < n, then ++*counter
__global__ void philox_uniforms_kernel(uint64_t seed, uint64_t* __restrict__ counter, int n, float* __restrict__ out) {
  const uint64_t ev = *counter;
  const int i = threadIdx.x;
  if (i < n) out[i] = philox_uniform(seed, ev, i);
  __syncthreads();                       // every thread has read the counter
  if (i == 0) *counter = ev + 1;
}

__global__ void gather_row_kernel(const uint16_t* __restrict__ src, long row_stride, const int32_t* __restrict__ idx,
                                  int rows, uint16_t* __restrict__ dst, int H) {
  int r = *idx;
  r = r < 0 ? 0 : (r >= rows ? rows - 1 : r);
  const uint16_t* s = src + (long)r * row_stride;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < H; i += gridDim.x * blockDim.x) dst[i] = s[i];
}

// ids[0] = *feed, ids[1 + i] = drafts[i]
__global__ void assemble_ids_kernel(const int32_t* __restrict__ feed, const int32_t* __restrict__ drafts, int k,
                                    int32_t* __restrict__ ids) {
  const int i = threadIdx.x;
  if (i == 0) ids[0] = *feed;
  else if (i <= k) ids[i] = drafts[i - 1];
}

// After the accept: pending ids [d_0 .. d_{n-1}, tok, 0 ...] (k + 1 slots),
// feed = tok, n_prev = n, out = [n, tok, d_0 .. d_{k-1}] for the host.
__global__ void cycle_finish_kernel(const int32_t* __restrict__ drafts, int k, const int32_t* __restrict__ n_ptr,
                                    const int32_t* __restrict__ tok_ptr, int32_t* __restrict__ pend_ids,
                                    int32_t* __restrict__ feed, int32_t* __restrict__ n_prev, int32_t* __restrict__ out) {
  const int i = threadIdx.x;
  const int n = *n_ptr, tok = *tok_ptr;
  if (i <= k) pend_ids[i] = i < n ? drafts[i] : (i == n ? tok : 0);
  if (i < k) out[2 + i] = drafts[i];
  if (i == 0) {
    *feed = tok;
    *n_prev = n;
    out[0] = n;
    out[1] = tok;
  }
}

// cycle_finish plus the rest of the cycle's bookkeeping in the same launch:
// ids_next[0] = tok (the next verify's first id), main_counters[i] += n + main_extra
// (the verify commit), mtp_counters[i] += mtp_delta (the draft steps' net
// advance), and u_out[i] = u(*u_counter, i), ++*u_counter (the next cycle's
// uniforms). Null pointers skip a part. Thread 0 writes all of `out`; with
// `done` it then makes those writes visible system-wide (a system-scope fence)
// and stores *done = 1, so a host that clears *done in pinned memory before the
// launch and polls it reads a complete result without a stream synchronisation.
__global__ void cycle_finish_ex_kernel(const int32_t* __restrict__ drafts, int k, const int32_t* __restrict__ n_ptr,
                                       const int32_t* __restrict__ tok_ptr, int32_t* __restrict__ pend_ids,
                                       int32_t* __restrict__ feed, int32_t* __restrict__ n_prev,
                                       int32_t* __restrict__ out, int32_t* __restrict__ ids_next,
                                       int32_t* __restrict__ main_counters, int n_main, int main_extra,
                                       int32_t* __restrict__ mtp_counters, int n_mtp, int mtp_delta,
                                       uint64_t u_seed, uint64_t* __restrict__ u_counter, int width,
                                       float* __restrict__ u_out, int32_t* __restrict__ done,
                                       const int32_t* __restrict__ rows) {
  const int i = threadIdx.x;
  // every read first, in one round trip (the counters' new values need only n)
  __shared__ int32_t sd[256];
  __shared__ int32_t srow[512];            // rows: 2 (k + 1) <= 512
  int32_t d = 0;
  if (i < k) d = drafts[i];
  if (i < k) sd[i] = d;
  if (rows && i < 2 * (k + 1)) srow[i] = rows[i];
  if (rows && i + 256 < 2 * (k + 1)) srow[i + 256] = rows[i + 256];
  const int32_t cm = (main_counters && i < n_main) ? main_counters[i] : 0;
  const int32_t ct = (mtp_counters && i < n_mtp) ? mtp_counters[i] : 0;
  const uint64_t ev = u_counter ? *u_counter : 0;
  const int n_given = rows ? 0 : *n_ptr, tok_given = rows ? 0 : *tok_ptr;
  __syncthreads();                       // every read of ids / the counter before the writes below
  int n, tok;
  if (rows) {
    // the verify rows' (accept flag, draw): the first rejected draft's draw, or
    // the bonus row's when all k are accepted
    n = k;
    for (int r = 0; r < k; ++r)
      if (!srow[2 * r]) {
        n = r;
        break;
      }
    tok = srow[2 * n + 1];
  } else {
    n = n_given;
    tok = tok_given;
  }
  if (i <= k) pend_ids[i] = i < n ? (i < k ? d : 0) : (i == n ? tok : 0);
  if (main_counters) {
    if (i < n_main) main_counters[i] = cm + n + main_extra;
    for (int c = i + (int)blockDim.x; c < n_main; c += blockDim.x) main_counters[c] += n + main_extra;
  }
  if (mtp_counters) {
    if (i < n_mtp) mtp_counters[i] = ct + mtp_delta;
    for (int c = i + (int)blockDim.x; c < n_mtp; c += blockDim.x) mtp_counters[c] += mtp_delta;
  }
  if (u_out && i < width) u_out[i] = philox_uniform(u_seed, ev, i);
  __syncthreads();
  if (i == 0) {
    *feed = tok;
    *n_prev = n;
    out[0] = n;
    out[1] = tok;
    for (int j = 0; j < k; ++j) out[2 + j] = sd[j];
    if (ids_next) ids_next[0] = tok;
    if (u_counter) *u_counter = ev + 1;
    if (done) {
      __threadfence_system();            // out[] (this thread's writes) before the flag
      __hip_atomic_store(done, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
  }
}

// seen[ids[q]] = 1 for q < min(max_ids, (n_ptr ? *n_ptr : 0) + n_offset); ids outside [0, V) skipped
__global__ void mark_seen_kernel(float* __restrict__ seen, int V, const int32_t* __restrict__ ids, int max_ids,
                                 const int32_t* __restrict__ n_ptr, int n_offset) {
  const int cnt = min(max_ids, (n_ptr ? *n_ptr : 0) + n_offset);
  for (int q = threadIdx.x; q < cnt; q += blockDim.x) {
    const int id = ids[q];
    if (id >= 0 && id < V) seen[id] = 1.0f;
  }
}

}  // namespace

extern "C" int qvex_mark_seen(float* seen, int V, const int32_t* ids, int max_ids, const int32_t* n_ptr,
                              int n_offset, void* stream) {
  QVEX_CHECK_ARG(seen && ids && V >= 1 && max_ids >= 0, "qvex_mark_seen: bad arguments");
  hipLaunchKernelGGL(mark_seen_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, seen, V, ids, max_ids, n_ptr,
                     n_offset);
  QVEX_CHECK_LAUNCH("qvex_mark_seen");
  return QVEX_OK;
}

extern "C" int qvex_gather_row(const uint16_t* src, long row_stride, const int32_t* idx, int rows, uint16_t* dst,
                               int H, void* stream) {
  QVEX_CHECK_ARG(src && idx && dst && rows >= 1 && H >= 1 && row_stride >= H, "qvex_gather_row: bad arguments");
  hipLaunchKernelGGL(gather_row_kernel, dim3((H + 255) / 256), dim3(256), 0, (hipStream_t)stream, src, row_stride,
                     idx, rows, dst, H);
  QVEX_CHECK_LAUNCH("qvex_gather_row");
  return QVEX_OK;
}

extern "C" int qvex_assemble_ids(const int32_t* feed, const int32_t* drafts, int k, int32_t* ids, void* stream) {
  QVEX_CHECK_ARG(feed && ids && (k == 0 || drafts) && k >= 0 && k < 256, "qvex_assemble_ids: bad arguments");
  hipLaunchKernelGGL(assemble_ids_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, feed, drafts, k, ids);
  QVEX_CHECK_LAUNCH("qvex_assemble_ids");
  return QVEX_OK;
}

extern "C" int qvex_cycle_finish(const int32_t* drafts, int k, const int32_t* n_accept, const int32_t* token,
                                 int32_t* pend_ids, int32_t* feed, int32_t* n_prev, int32_t* out, void* stream) {
  QVEX_CHECK_ARG(drafts && n_accept && token && pend_ids && feed && n_prev && out && k >= 1 && k < 255,
                 "qvex_cycle_finish: bad arguments");
  hipLaunchKernelGGL(cycle_finish_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, drafts, k, n_accept, token,
                     pend_ids, feed, n_prev, out);
  QVEX_CHECK_LAUNCH("qvex_cycle_finish");
  return QVEX_OK;
}

extern "C" int qvex_philox_uniforms(uint64_t seed, uint64_t* counter, int n, float* out, void* stream) {
  QVEX_CHECK_ARG(counter && out && n >= 1 && n <= 256, "qvex_philox_uniforms: bad arguments (n=%d, 1..256)", n);
  hipLaunchKernelGGL(philox_uniforms_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, seed, counter, n, out);
  QVEX_CHECK_LAUNCH("qvex_philox_uniforms");
  return QVEX_OK;
}

extern "C" int qvex_cycle_finish_ex(const int32_t* drafts, int k, const int32_t* n_accept, const int32_t* token,
                                    int32_t* pend_ids, int32_t* feed, int32_t* n_prev, int32_t* out,
                                    int32_t* ids_next, int32_t* main_counters, int n_main, int main_extra,
                                    int32_t* mtp_counters, int n_mtp, int mtp_delta, uint64_t u_seed,
                                    uint64_t* u_counter, int u_width, float* u_out, int32_t* done,
                                    const int32_t* rows, void* stream) {
  QVEX_CHECK_ARG(drafts && (rows || (n_accept && token)) && pend_ids && feed && n_prev && out && k >= 1 && k < 255,
                 "qvex_cycle_finish_ex: bad arguments");
  QVEX_CHECK_ARG((!main_counters || n_main >= 0) && (!mtp_counters || n_mtp >= 0) &&
                     (!u_out || (u_counter && u_width >= 1 && u_width <= 256)),
                 "qvex_cycle_finish_ex: bad counter or uniform arguments");
  hipLaunchKernelGGL(cycle_finish_ex_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, drafts, k, n_accept, token,
                     pend_ids, feed, n_prev, out, ids_next, main_counters, n_main, main_extra, mtp_counters, n_mtp,
                     mtp_delta, u_seed, u_counter, u_width, u_out, done, rows);
  QVEX_CHECK_LAUNCH("qvex_cycle_finish_ex");
  return QVEX_OK;
}
