/*
 * gq_sample.hip — sampling the next token on the device from logits already
 * there (the LM head's output), so a sampled decode step needs no logits
 * round trip (tokenizer.c:175-333 on the host copies 501 KiB per token at
 * the 8B shape).
 *
 * The reference draws one rand() per sampled token and scales it as
 * (float)rand() / (float)RAND_MAX (temperature, top-k) or in double
 * (top-p).  The caller passes that raw draw (`rnd`), so with the same libc
 * stream the device sees the same random numbers.
 *
 *   top-k (tokenizer.c:219-280): the reference keeps k slots, filled with
 *     logits 0..k-1, and for every later logit above the slots' minimum
 *     replaces that minimum (the lowest slot among equal minima).  The
 *     slots' order decides which token a given draw picks, so the kernel
 *     replays exactly that insertion sequence: logits 0..kPre-1 by one
 *     wave, 64 at a time, then every later logit above the minimum after
 *     kPre (the running minimum only rises, so nothing below it can be
 *     inserted later), gathered by all waves and inserted in index order.
 *     For k <= 64 the slots live in registers, one per lane, and a
 *     replacement's new minimum is one DPP reduction.  The softmax over the
 *     slots and the draw then run on one thread in the reference's order.
 *   top-p (tokenizer.c:282-333): stable descending sort (rocPRIM's device
 *     radix sort of (logit, index) pairs; the reference's qsort is glibc's
 *     merge sort, stable for equal logits),
 *     then the cumulative probabilities in double.
 *   temperature (tokenizer.c:187-217): the exponentials in parallel, the
 *     reference's sequential float sum and scan on one thread (see
 *     temp_kernel).
 */
#include <rocprim/device/device_radix_sort.hpp>

#include "gq_device.h"
#include "gq_internal.h"

namespace {

constexpr int kST = 1024;           /* threads of the one-workgroup kernels */
constexpr int kSW = kST / GQ_WAVE;  /* their waves */
constexpr int kPre = 4 * kST;       /* logits replayed chunk by chunk before the filter */
constexpr int kCandCap = 8192;      /* filtered candidates held in LDS */
constexpr float kRandMax = 2147483647.0f; /* RAND_MAX of glibc, as the reference casts it */

/* A float's bits mapped to an unsigned integer of the same order. */
__device__ __forceinline__ uint32_t ord_bits(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

/* 64-bit DPP move of the row operation CTRL (rows not in RM keep their own
 * value) */
template <int CTRL, int RM>
__device__ __forceinline__ uint64_t dpp64(uint64_t k) {
  const int lo = (int)(uint32_t)k, hi = (int)(uint32_t)(k >> 32);
  const uint32_t nlo = (uint32_t)__builtin_amdgcn_update_dpp(lo, lo, CTRL, RM, 0xf, false);
  const uint32_t nhi = (uint32_t)__builtin_amdgcn_update_dpp(hi, hi, CTRL, RM, 0xf, false);
  return ((uint64_t)nhi << 32) | nlo;
}

/* The wave's smallest 64-bit key, in every lane: quad swaps, half-row and
 * row mirrors, then the row broadcasts 15 and 31 into lane 63. */
__device__ __forceinline__ uint64_t wave_min_key(uint64_t k) {
  uint64_t t;
  t = dpp64<0xb1, 0xf>(k), k = t < k ? t : k; /* quad_perm [1,0,3,2] */
  t = dpp64<0x4e, 0xf>(k), k = t < k ? t : k; /* quad_perm [2,3,0,1] */
  t = dpp64<0x141, 0xf>(k), k = t < k ? t : k; /* row_half_mirror */
  t = dpp64<0x140, 0xf>(k), k = t < k ? t : k; /* row_mirror */
  t = dpp64<0x142, 0xa>(k), k = t < k ? t : k; /* row_bcast:15 */
  t = dpp64<0x143, 0xc>(k), k = t < k ? t : k; /* row_bcast:31 */
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)k, 63);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(k >> 32), 63);
  return ((uint64_t)hi << 32) | lo;
}

/* (value, slot) of the slots' minimum with the reference's tie rule (the
 * first slot holding the smallest value), over slots [0, k), by one wave:
 * the minimum of (value order, slot) keys */
__device__ void wave_min(const float *tv, int k, int lane, float &mv, int &mj) {
  uint64_t key = ~0ull;
  for (int s = lane; s < k; s += GQ_WAVE) {
    const float t = tv[s];
    const uint64_t c = ((uint64_t)ord_bits(t == 0.f ? 0.f : t) << 32) | (uint32_t)s; /* -0 equals +0 */
    key = c < key ? c : key;
  }
  key = wave_min_key(key);
  mj = (int)(uint32_t)key;
  mv = tv[mj];
}

/* inverse of ord_bits */
__device__ __forceinline__ float from_ord(uint32_t o) {
  return __builtin_bit_cast(float, (o & 0x80000000u) ? (o ^ 0x80000000u) : ~o);
}

/* The k slots of the reference's top-k, held by wave 0.  k <= 64: one slot
 * per lane in registers; larger k: in LDS. */
struct RegSlots {
  float v;
  int i, k, lane;
  __device__ void init(const float *x, int k_, int lane_) {
    k = k_, lane = lane_;
    v = lane < k ? x[lane] : 0.f;
    i = lane;
  }
  /* the minimum with the reference's tie rule (first slot of the smallest) */
  __device__ void minimum(float &mv, int &mj) const {
    const uint64_t key = lane < k ? ((uint64_t)ord_bits(v == 0.f ? 0.f : v) << 32) | (uint32_t)lane : ~0ull;
    const uint64_t m = wave_min_key(key);
    mj = (int)(uint32_t)m;
    mv = from_ord((uint32_t)(m >> 32));
  }
  __device__ void replace(int mj, float nv, int ni) {
    if (lane == mj) v = nv, i = ni;
  }
  __device__ void store(float *tv, int *ti) const {
    if (lane < k) tv[lane] = v, ti[lane] = i;
  }
};

struct LdsSlots {
  float *tv;
  int *ti;
  int k, lane;
  __device__ void init(const float *x, int k_, int lane_) {
    k = k_, lane = lane_;
    for (int j = lane; j < k; j += GQ_WAVE) tv[j] = x[j], ti[j] = j;
    __builtin_amdgcn_s_waitcnt(0xc07f); /* lgkmcnt(0) */
    __builtin_amdgcn_wave_barrier();
  }
  __device__ void minimum(float &mv, int &mj) const { wave_min(tv, k, lane, mv, mj); }
  __device__ void replace(int mj, float nv, int ni) {
    if (lane == 0) tv[mj] = nv, ti[mj] = ni;
    __builtin_amdgcn_s_waitcnt(0xc07f); /* the slot write lands before the rescan */
    __builtin_amdgcn_wave_barrier();
  }
  __device__ void store(float *, int *) const {}
};

/* Wave 0 replays the reference's slot updates for a group of up to 64
 * candidates held one per lane in index order (valid lanes flagged). */
template <class S>
__device__ __forceinline__ void insert_lanes(S &sl, bool valid, float v, int id, float &mv, int &mj) {
  const int lane = sl.lane;
  uint64_t live = __ballot(valid && v > mv);
  while (live) {
    const int l = __builtin_ctzll(live); /* the next candidate in index order */
    const float vl = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
    const int il = __builtin_amdgcn_readlane(id, l);
    sl.replace(mj, vl, il);
    sl.minimum(mv, mj);
    live = __ballot(valid && lane > l && v > mv);
  }
}

/* Wave 0 over logits [lo, hi) in index order, 64 at a time (the next 64
 * already loading) */
template <class S>
__device__ void scan_range(S &sl, const float *x, int lo, int hi, float &mv, int &mj) {
  const int lane = sl.lane;
  float nx = lo + lane < hi ? x[lo + lane] : 0.f;
  for (int b = lo; b < hi; b += GQ_WAVE) {
    const float v = nx;
    nx = b + GQ_WAVE + lane < hi ? x[b + GQ_WAVE + lane] : 0.f;
    insert_lanes(sl, b + lane < hi, v, b + lane, mv, mj);
  }
}

struct TopkShared {
  float tv[kMaxTopK], pr[kMaxTopK];
  int ti[kMaxTopK];
  int ci[kCandCap];
  float cv[kCandCap];
  int wn[kSW], wovf[kSW];
  float s_mv;
  int s_mj;
};

template <class S>
__device__ void topk_body(S &sl, const float *x, int V, int k, float T, int rnd, int *out, TopkShared &sh) {
  float *tv = sh.tv, *pr = sh.pr, *cv = sh.cv;
  int *ti = sh.ti, *ci = sh.ci, *wn = sh.wn, *wovf = sh.wovf;
  float &s_mv = sh.s_mv;
  int &s_mj = sh.s_mj;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  /* logits 0 .. pre-1 by wave 0 alone: the slots' first k, then in order */
  const int pre = min(V, max(kPre, k));
  if (wave == 0) {
    float mv;
    int mj;
    sl.init(x, k, lane);
    sl.minimum(mv, mj);
    scan_range(sl, x, k, pre, mv, mj);
    if (lane == 0) s_mv = mv, s_mj = mj;
  }
  __syncthreads();
  /* the rest: each wave gathers, in index order, the logits of its own
   * contiguous slice above the minimum after `pre` logits (the minimum only
   * rises, so no other logit can enter a slot later); a wave whose list
   * fills up records where it stopped */
  const float thr = s_mv;
  constexpr int kCapW = kCandCap / kSW;
  const int per = (V - pre + kSW - 1) / kSW, lo = min(V, pre + wave * per), hi = min(V, lo + per);
  int n = 0, ovf = hi;
  for (int b0 = lo; b0 < hi && ovf == hi; b0 += 8 * GQ_WAVE) {
    float vv[8]; /* eight groups' loads in flight at once */
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const int i = b0 + u * GQ_WAVE + lane;
      vv[u] = i < hi ? x[i] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const int b = b0 + u * GQ_WAVE, i = b + lane;
      const bool c = i < hi && vv[u] > thr;
      const uint64_t bal = __ballot(c);
      const int cnt = __popcll(bal);
      if (ovf == hi && b < hi) {
        if (n + cnt > kCapW) {
          ovf = b;
        } else {
          const int at = n + __popcll(bal & ((1ull << lane) - 1ull));
          if (c) ci[wave * kCapW + at] = i, cv[wave * kCapW + at] = vv[u];
          n += cnt;
        }
      }
    }
  }
  if (lane == 0) wn[wave] = n, wovf[wave] = ovf;
  __syncthreads();
  /* wave 0: the gathered lists in order up to the first slice that filled
   * up, then logit by logit from there */
  if (wave == 0) {
    float mv = s_mv;
    int mj = s_mj;
    int resume = V;
    for (int w = 0; w < kSW; w++) {
      for (int q0 = 0; q0 < wn[w]; q0 += GQ_WAVE) {
        const int q = q0 + lane;
        const bool ok = q < wn[w];
        insert_lanes(sl, ok, ok ? cv[w * kCapW + q] : 0.f, ok ? ci[w * kCapW + q] : 0, mv, mj);
      }
      const int whi = min(V, min(V, pre + w * per) + per);
      if (wovf[w] < whi) {
        resume = wovf[w];
        break;
      }
    }
    if (resume < V) scan_range(sl, x, resume, V, mv, mj);
    sl.store(tv, ti);
  }
  __syncthreads();
  /* temperature softmax over the slots and the draw, in the reference's
   * order (tokenizer.c:254-276) */
  if (tid == 0) {
    float mx = tv[0];
    for (int j = 1; j < k; j++)
      if (tv[j] > mx) mx = tv[j];
    float sum = 0.f;
    for (int j = 0; j < k; j++) {
      const float p = expf((tv[j] - mx) / T);
      pr[j] = p;
      sum += p;
    }
    const float r = ((float)rnd / kRandMax) * sum;
    float acc = 0.f;
    int pick = k - 1;
    for (int j = 0; j < k; j++) {
      acc += pr[j];
      if (r <= acc) {
        pick = j;
        break;
      }
    }
    *out = ti[pick];
  }
}

__global__ __launch_bounds__(kST) void topk_kernel(const float *x, int V, int k, float T, int rnd, int *out) {
  __shared__ TopkShared sh;
  if (k <= GQ_WAVE) {
    RegSlots sl;
    topk_body(sl, x, V, k, T, rnd, out, sh);
  } else {
    LdsSlots sl;
    sl.tv = sh.tv, sl.ti = sh.ti;
    topk_body(sl, x, V, k, T, rnd, out, sh);
  }
}

/* Block-wide exclusive scan of one double per thread; returns the prefix,
 * *total gets the sum (all threads). */
__device__ double block_scan(double v, double *total, double *sw) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  double inc = v;
#pragma unroll
  for (int o = 1; o < GQ_WAVE; o <<= 1) {
    const double t = __shfl_up(inc, o);
    if (lane >= o) inc += t;
  }
  if (lane == GQ_WAVE - 1) sw[wave] = inc;
  __syncthreads();
  double off = 0.0, tot = 0.0;
#pragma unroll
  for (int w = 0; w < kSW; w++) {
    off += w < wave ? sw[w] : 0.0;
    tot += sw[w];
  }
  __syncthreads();
  *total = tot;
  return off + inc - v;
}

__device__ float block_max(float v, float *sw) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = gq_wave_max(v);
  if (lane == 0) sw[wave] = v;
  __syncthreads();
  float m = sw[0];
#pragma unroll
  for (int w = 1; w < kSW; w++) m = fmaxf(m, sw[w]);
  __syncthreads();
  return m;
}

/* The first index i in [0, n) whose inclusive running sum of w(i) reaches r
 * (n - 1 when none does); w(i) summed in double, each thread over one
 * contiguous segment. */
template <typename W>
__device__ int first_reaching(W w, int n, double r, double *sw, int *s_pick) {
  const int tid = threadIdx.x, seg = (n + kST - 1) / kST, lo = min(tid * seg, n), hi = min(lo + seg, n);
  double part = 0.0;
  for (int i = lo; i < hi; i++) part += w(i);
  double tot;
  const double before = block_scan(part, &tot, sw);
  if (tid == 0) *s_pick = n - 1;
  __syncthreads();
  if (before < r && r <= before + part) {
    /* the running sum reaches r inside this segment (its last element when
     * the sequential sum rounds just below before + part) */
    double acc = before;
    int found = hi - 1;
    for (int i = lo; i < hi; i++) {
      acc += w(i);
      if (r <= acc) {
        found = i;
        break;
      }
    }
    atomicMin(s_pick, found);
  } else if (r <= before && tid == 0) {
    atomicMin(s_pick, 0);
  }
  __syncthreads();
  return *s_pick;
}

/* softmax(x / T) over the vocabulary and one draw (tokenizer.c:187-217).
 * The reference sums the probabilities sequentially in float, and over a
 * large vocabulary that sum's rounding moves the cumulative boundaries by
 * far more than a last bit (a double sum picks a different token for about
 * one draw in four at 128256 entries), so the two sequential loops run as
 * written, on one thread: the workgroup computes the exponentials in
 * parallel and stages them through LDS in chunks of kChunkP. */
constexpr int kChunkP = 32768;

constexpr int kCkMax = 4096; /* 64-entry blocks: vocabularies up to 262144 */

__global__ __launch_bounds__(kST) void temp_kernel(const float *x, int V, float T, int rnd, float *prob, int *out) {
  __shared__ float sf[kSW];
  __shared__ float chunk[kChunkP];
  __shared__ float ck[kCkMax + 1]; /* running sum before each 64-entry block, then the total */
  __shared__ float s_r;
  __shared__ int s_blk, s_pick;
  const int tid = threadIdx.x;
  float m = -INFINITY;
  for (int i = tid; i < V; i += kST) m = fmaxf(m, x[i]);
  const float mx = block_max(m, sf);
  for (int i = tid; i < V; i += kST) prob[i] = expf((x[i] - mx) / T);
  /* the reference's running float sum, one thread, its value recorded at
   * the start of every 64-entry block */
  float sum = 0.f;
  for (int base = 0; base < V; base += kChunkP) {
    const int n = min(kChunkP, V - base);
    __syncthreads();
    for (int i = tid; i < n; i += kST) chunk[i] = prob[base + i];
    __syncthreads();
    if (tid == 0)
      for (int b = 0; b < n; b += 64) {
        ck[(base + b) >> 6] = sum;
        const int e = min(64, n - b);
        if (e == 64) {
#pragma unroll
          for (int j = 0; j < 64; j++) sum += chunk[b + j];
        } else {
          for (int j = 0; j < e; j++) sum += chunk[b + j];
        }
      }
  }
  const int nblk = (V + 63) >> 6;
  if (tid == 0) ck[nblk] = sum, s_r = ((float)rnd / kRandMax) * sum, s_blk = nblk, s_pick = V - 1;
  __syncthreads();
  /* the first block whose closing sum reaches r (sums never decrease) ... */
  const float r = s_r;
  for (int q = tid; q < nblk; q += kST)
    if (r <= ck[q + 1]) {
      atomicMin(&s_blk, q);
      break;
    }
  __syncthreads();
  /* ... then its 64 additions again, from its opening sum */
  if (tid == 0 && s_blk < nblk) {
    float acc = ck[s_blk];
    const int lo = s_blk << 6, hi = min(lo + 64, V);
    for (int i = lo; i < hi; i++) {
      acc += prob[i];
      if (r <= acc) {
        s_pick = i;
        break;
      }
    }
  }
  __syncthreads();
  if (tid == 0) *out = s_pick;
}

/* top-p over the logits sorted in descending order (keys) with their token
 * ids (ids), tokenizer.c:296-333 */
__global__ __launch_bounds__(kST) void topp_kernel(const float *keys, const int *ids, int V, float p, float T, int rnd,
                                                    int *out) {
  __shared__ double sw[kSW];
  __shared__ int s_pick;
  const float mx = keys[0];
  auto w = [&](int i) { return (double)expf((keys[i] - mx) / T); };
  double tot = 0.0;
  {
    const int seg = (V + kST - 1) / kST, lo = min((int)threadIdx.x * seg, V), hi = min(lo + seg, V);
    double part = 0.0;
    for (int i = lo; i < hi; i++) part += w(i);
    (void)block_scan(part, &tot, sw);
  }
  /* cutoff: how many leading tokens until the cumulative share reaches p */
  const double tot_c = tot;
  auto share = [&](int i) { return w(i) / tot_c; };
  const int cutoff = first_reaching(share, V, (double)p, sw, &s_pick) + 1;
  /* the draw over the first `cutoff` tokens */
  double cut = 0.0;
  {
    const int seg = (cutoff + kST - 1) / kST, lo = min((int)threadIdx.x * seg, cutoff), hi = min(lo + seg, cutoff);
    double part = 0.0;
    for (int i = lo; i < hi; i++) part += w(i);
    (void)block_scan(part, &cut, sw);
  }
  const double r = ((double)rnd / 2147483647.0) * cut;
  const int pick = first_reaching(w, cutoff, r, sw, &s_pick);
  if (threadIdx.x == 0) *out = ids[pick];
}

__global__ void iota_kernel(int *v, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) v[i] = i;
}

} // namespace

size_t gq_sample_ws_bytes(int vocab) {
  size_t bytes = 0;
  (void)rocprim::radix_sort_pairs_desc(nullptr, bytes, (const float *)nullptr, (float *)nullptr,
                                       (const int *)nullptr, (int *)nullptr, (size_t)vocab);
  return bytes;
}

int gq_launch_sample(const float *logits, int vocab, float temperature, int top_k, float top_p, int rnd,
                     const SampleWs &ws, int *out, hipStream_t s) {
  if (vocab <= 0 || !logits || !out) return -1;
  if (temperature <= 0.0f) return 1; /* greedy: the argmax path */
  if (top_k > 0 && top_k < vocab) {
    if (top_k > kMaxTopK) return -2;
    hipLaunchKernelGGL(topk_kernel, dim3(1), dim3(kST), 0, s, logits, vocab, top_k, temperature, rnd, out);
  } else if (top_p < 1.0f) {
    if (top_p <= 0.0f) return 1; /* greedy (tokenizer.c:287) */
    if (!ws.keys || !ws.ids_in || !ws.ids || !ws.sort_tmp || ws.cap < vocab) return -1;
    hipLaunchKernelGGL(iota_kernel, dim3((vocab + 255) / 256), dim3(256), 0, s, ws.ids_in, vocab);
    size_t bytes = ws.sort_bytes;
    if (rocprim::radix_sort_pairs_desc(ws.sort_tmp, bytes, logits, ws.keys, ws.ids_in, ws.ids, (size_t)vocab, 0,
                                       8 * (unsigned)sizeof(float), s) != hipSuccess)
      return -4;
    hipLaunchKernelGGL(topp_kernel, dim3(1), dim3(kST), 0, s, ws.keys, ws.ids, vocab, top_p, temperature, rnd, out);
  } else {
    if (!ws.keys || ws.cap < vocab || vocab > 64 * kCkMax) return -1;
    hipLaunchKernelGGL(temp_kernel, dim3(1), dim3(kST), 0, s, logits, vocab, temperature, rnd, ws.keys, out);
  }
  return hipGetLastError() == hipSuccess ? 0 : -4;
}
