// Token sampling on the device: Sampler.sample(logits:) (Sources/AlpacaCore/
// Runtime/Sampler.swift:57-93) for a draw u in [0, 1) supplied by the caller's
// RNG, so a step's logits never leave HBM.
//
// The reference: temperature 0 is the arg-max (lowest index on ties; NaN is an
// error).  Otherwise NaN is an error; top-k keeps the k largest logits (ties to
// the lower index); p_i = exp((l_i - top) / t) in double; top-p keeps the
// shortest prefix whose cumulative p/sum reaches top_p; the draw walks the kept
// probabilities in order until their running sum exceeds u * sum.  Candidates
// are in logit-descending, index-ascending order when top-k or top-p applies,
// in index order otherwise.
//
// One workgroup of 1024 threads:
//   * plain temperature (no top-k, top-p = 1): each thread sums the
//     probabilities of a contiguous chunk of indices, thread 0 combines the
//     chunk sums in order and walks the chunk that holds the draw.  The sums
//     are associated by chunk rather than strictly left to right, so the token
//     can differ from a strictly sequential sum only when u * sum falls within
//     about 1e-16 (relative) of a boundary between two tokens.
//   * top-k and/or top-p: candidates are produced in the reference's order in
//     windows of up to 1024, each the next smallest (key, index) pairs after
//     the previous window: a radix select over the 32-bit order key (4 passes
//     of 8 bits, LDS histograms), the boundary's tied indices taken in index
//     order, a gather and a bitonic sort in LDS.  Their indices and
//     probabilities go to a scratch list, and thread 0 accumulates the sums in
//     exactly the reference's order: the top-k total, the top-p cumulative of
//     p/sum, the kept total and the draw.  Without top-k the total for top-p is
//     a chunked sum over all logits (same caveat as above).  Most draws need
//     one window; a flat distribution under top-p may need many.
#include "common.h"

#include <limits.h>

namespace {

constexpr int kST = 1024;  // threads
constexpr int kWin = 1024;  // candidates per window

struct SampleArgs {
    const float* logits;
    int n;
    float temperature;
    int top_k;
    float top_p;
    double u;
    int32_t* out;       // [1] token
    int* status;        // [1] 0 ok, 1 NaN in the logits
    uint32_t* cand_idx;  // [n] scratch: candidate indices in order
    double* cand_p;      // [n] scratch: their probabilities
};

// Ascending in this key = logit descending; -0 and +0 share a key (they compare equal).
__device__ __forceinline__ uint32_t order_key(float l) {
    if (l == 0.0f) l = 0.0f;
    const uint32_t u = __float_as_uint(l);
    const uint32_t asc = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ~asc;
}
__device__ __forceinline__ uint64_t composite(uint32_t key, uint32_t idx) { return ((uint64_t)key << 32) | idx; }

__device__ __forceinline__ double prob(float l, double top, double t) { return exp(((double)l - top) / t); }

}  // namespace

__global__ __launch_bounds__(kST) void sample_kernel(SampleArgs a) {
    __shared__ int s_int[32];
    __shared__ float s_f[32];
    __shared__ double s_d[kST];        // chunk sums
    __shared__ uint32_t s_hist[256];
    __shared__ uint64_t s_win[kWin];   // window being sorted
    __shared__ uint32_t s_tie[kST];    // per-thread tie counts
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, n = a.n;
    const float* L = a.logits;

    // ---- NaN check and maximum (lowest index on ties for the arg-max)
    float mx = -INFINITY;
    int mi = INT_MAX, nan = 0;
    for (int i = tid; i < n; i += kST) {
        const float l = L[i];
        if (l != l) nan = 1;
        else if (l > mx || mi == INT_MAX) {  // a thread's indices ascend: later equal values never win
            mx = l;
            mi = i;
        }
    }
    for (int o = 32; o > 0; o >>= 1) {
        const float m2 = __shfl_xor(mx, o, 64);
        const int i2 = __shfl_xor(mi, o, 64);
        if (m2 > mx || (m2 == mx && i2 < mi)) {
            mx = m2;
            mi = i2;
        }
        nan |= __shfl_xor(nan, o, 64);
    }
    if (lane == 0) {
        s_f[wave] = mx;
        s_int[wave] = mi;
        s_int[16 + wave] = nan;
    }
    __syncthreads();
    if (tid == 0) {
        float bm = s_f[0];
        int bi = s_int[0], bn = s_int[16];
        for (int w = 1; w < kST / 64; w++) {
            if (s_f[w] > bm || (s_f[w] == bm && s_int[w] < bi)) {
                bm = s_f[w];
                bi = s_int[w];
            }
            bn |= s_int[16 + w];
        }
        s_f[16] = bm;
        s_int[30] = bi;
        s_int[31] = bn;
    }
    __syncthreads();
    if (s_int[31]) {
        if (tid == 0) {
            *a.status = 1;
            *a.out = -1;
        }
        return;
    }
    if (a.temperature == 0.0f) {  // Sampler.argmax
        if (tid == 0) {
            *a.status = 0;
            *a.out = s_int[30];
        }
        return;
    }
    const double top = (double)s_f[16], t = (double)a.temperature;
    const int K = a.top_k > 0 ? min(a.top_k, n) : n;
    const bool sorted = K < n || a.top_p < 1.0f;
    const int chunk = (n + kST - 1) / kST, c0 = min(n, tid * chunk), c1 = min(n, c0 + chunk);

    // Sum of all probabilities by index chunks, combined in chunk order.
    auto chunked_total = [&]() -> double {
        double s = 0.0;
        for (int i = c0; i < c1; i++) s += prob(L[i], top, t);
        s_d[tid] = s;
        __syncthreads();
        if (tid == 0) {
            double tot = 0.0;
            for (int k = 0; k < kST; k++) tot += s_d[k];
            s_d[0] = tot;  // chunk 0's own sum is no longer needed once combined
        }
        __syncthreads();
        const double tot = s_d[0];
        __syncthreads();
        return tot;
    };

    if (!sorted) {
        // chunk sums in order, then the chunk holding the draw, walked left to right
        double s = 0.0;
        for (int i = c0; i < c1; i++) s += prob(L[i], top, t);
        s_d[tid] = s;
        __syncthreads();
        if (tid == 0) {
            double tot = 0.0;
            for (int k = 0; k < kST; k++) tot += s_d[k];
            const double target = a.u * tot;
            double acc = 0.0;
            int token = n - 1;
            for (int k = 0; k < kST; k++) {
                const int b0 = min(n, k * chunk), b1 = min(n, b0 + chunk);
                if (b0 >= b1) continue;
                if (target < acc + s_d[k]) {
                    double a2 = acc;
                    for (int i = b0; i < b1; i++) {
                        a2 += prob(L[i], top, t);
                        if (target < a2) {
                            token = i;
                            break;
                        }
                    }
                    if (a2 > target) break;  // found (else rounding left it past the chunk: continue)
                }
                acc += s_d[k];
            }
            *a.status = 0;
            *a.out = token;
        }
        return;
    }

    // ---- sorted candidates, produced window by window
    int produced = 0;      // candidates in the scratch list
    bool have_prev = false;
    uint64_t prev = 0;     // composite of the last candidate produced

    // Appends the next m candidates (m <= kWin, m <= n - produced) in order.
    auto next_window = [&](int m) {
        uint32_t prefix = 0, mask = 0;
        int need = m;
        for (int pass = 0; pass < 4; pass++) {
            const int shift = 24 - 8 * pass;
            for (int b = tid; b < 256; b += kST) s_hist[b] = 0;
            __syncthreads();
            for (int i = tid; i < n; i += kST) {
                const uint32_t key = order_key(L[i]);
                if (have_prev && composite(key, (uint32_t)i) <= prev) continue;
                if ((key & mask) != prefix) continue;
                atomicAdd(&s_hist[(key >> shift) & 255u], 1u);
            }
            __syncthreads();
            if (tid == 0) {
                int cum = 0, b = 0;
                for (; b < 255; b++) {
                    if (cum + (int)s_hist[b] >= need) break;
                    cum += (int)s_hist[b];
                }
                s_int[0] = b;
                s_int[1] = need - cum;
            }
            __syncthreads();
            prefix |= (uint32_t)s_int[0] << shift;
            mask |= 255u << shift;
            need = s_int[1];
            __syncthreads();
        }
        // `prefix` is the boundary key; take its `need` lowest-index members (after prev)
        const uint32_t bkey = prefix;
        uint32_t ties = 0;
        for (int i = c0; i < c1; i++) {
            const uint32_t key = order_key(L[i]);
            if (key == bkey && !(have_prev && composite(key, (uint32_t)i) <= prev)) ties++;
        }
        s_tie[tid] = ties;
        __syncthreads();
        if (tid == 0) {
            int cum = 0, k = 0;
            for (; k < kST; k++) {
                if (cum + (int)s_tie[k] >= need) break;
                cum += (int)s_tie[k];
            }
            // walk chunk k for the (need - cum)-th tied index
            int left = need - cum, bidx = -1;
            const int b0 = min(n, k * chunk), b1 = min(n, b0 + chunk);
            for (int i = b0; i < b1 && left > 0; i++) {
                const uint32_t key = order_key(L[i]);
                if (key == bkey && !(have_prev && composite(key, (uint32_t)i) <= prev) && --left == 0) bidx = i;
            }
            s_int[2] = bidx;
            s_int[3] = 0;  // gather counter
        }
        __syncthreads();
        const uint64_t bound = composite(bkey, (uint32_t)s_int[2]);
        for (int i = tid; i < n; i += kST) {
            const uint64_t c = composite(order_key(L[i]), (uint32_t)i);
            if ((have_prev && c <= prev) || c > bound) continue;
            const int slot = atomicAdd(&s_int[3], 1);
            if (slot < kWin) s_win[slot] = c;  // exactly m <= kWin pass: the passes count the same elements
        }
        __syncthreads();
        for (int k = m + tid; k < kWin; k += kST) s_win[k] = ~0ull;  // padding sorts last
        __syncthreads();
        // bitonic sort of kWin composites, ascending
        for (int size = 2; size <= kWin; size <<= 1)
            for (int stride = size >> 1; stride > 0; stride >>= 1) {
                for (int k = tid; k < kWin; k += kST) {
                    const int j = k ^ stride;
                    if (j > k) {
                        const uint64_t x = s_win[k], y = s_win[j];
                        const bool up = (k & size) == 0;
                        if ((x > y) == up) {
                            s_win[k] = y;
                            s_win[j] = x;
                        }
                    }
                }
                __syncthreads();
            }
        for (int k = tid; k < m; k += kST) {
            const uint32_t idx = (uint32_t)(s_win[k] & 0xFFFFFFFFu);
            a.cand_idx[produced + k] = idx;
            a.cand_p[produced + k] = prob(L[idx], top, t);
        }
        prev = s_win[m - 1];
        have_prev = true;
        produced += m;
        __syncthreads();  // the scratch list is complete for thread 0
    };

    // total over the candidates: the top-k prefix in order, or every logit by chunks
    double total = 0.0;
    if (K < n) {
        while (produced < K) next_window(min(kWin, K - produced));
        if (tid == 0) {
            double s = 0.0;
            for (int i = 0; i < K; i++) s += a.cand_p[i];
            s_d[0] = s;
        }
        __syncthreads();
        total = s_d[0];
        __syncthreads();
    } else {
        total = chunked_total();
    }

    // top-p: the shortest prefix whose cumulative p/total reaches top_p, and its sum
    int keep = K;
    double kept = total;
    if (a.top_p < 1.0f) {
        int walked = 0;
        double cum = 0.0;
        while (true) {
            if (walked == produced) {
                if (produced == K) break;
                next_window(min(kWin, K - produced));
            }
            if (tid == 0) {
                int found = -1;
                for (int i = walked; i < produced; i++) {
                    cum += a.cand_p[i] / total;
                    if (cum >= (double)a.top_p) {
                        found = i + 1;
                        break;
                    }
                }
                s_int[4] = found;
            }
            __syncthreads();
            const int found = s_int[4];
            __syncthreads();
            if (found > 0) {
                keep = found;
                break;
            }
            walked = produced;
        }
        // the kept total, summed afresh in order (Sampler.swift:79)
        if (tid == 0) {
            double s = 0.0;
            for (int i = 0; i < keep; i++) s += a.cand_p[i];
            s_d[0] = s;
        }
        __syncthreads();
        kept = s_d[0];
        __syncthreads();
    }

    // the draw
    if (tid == 0) {
        const double target = a.u * kept;
        double acc = 0.0;
        int token = (int)a.cand_idx[keep - 1];
        for (int i = 0; i < keep; i++) {
            acc += a.cand_p[i];
            if (target < acc) {
                token = (int)a.cand_idx[i];
                break;
            }
        }
        *a.status = 0;
        *a.out = token;
    }
}

hipError_t launch_sample(const float* logits, int n, float temperature, int top_k, float top_p, double u,
                         int32_t* out, int* status, uint32_t* cand_idx, double* cand_p, hipStream_t st) {
    if (n <= 0) return hipErrorInvalidValue;
    SampleArgs a{logits, n, temperature, top_k, top_p, u, out, status, cand_idx, cand_p};
    sample_kernel<<<1, kST, 0, st>>>(a);
    return hipGetLastError();
}
