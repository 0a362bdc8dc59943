// shim.hip — the extern "C" boundary of libtqhip.so (declared in
// include/tq/tq_hip.h): device selection, error mapping, the paged KV cache
// object, split-K planning, synchronous host-buffer entry points and async
// device-buffer entry points.  No entry point aborts; HIP errors come back as
// TQ_HIP_EHIP_BASE - hipError_t.
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include <algorithm>
#include <mutex>
#include <new>
#include <vector>

#include "tq_common.hpp"

struct tq_hip_kv {
    tq_hip_kv_desc desc;
    int device = 0;
    hipStream_t stream = nullptr;
    unsigned char *pool = nullptr;
    size_t pool_bytes = 0;
    int32_t *d_page_table = nullptr;
    std::vector<int32_t> h_page_table;
    tq::PagedView view{};
    float *partials = nullptr;      // split-K scratch, grown on demand
    size_t partials_bytes = 0;
    int *counters = nullptr;        // split-K arrival counters, zero between launches
    size_t counters_n = 0;
    unsigned char *stage = nullptr; // device staging for the synchronous calls
    unsigned char *hstage = nullptr;  // its pinned host mirror: one copy in, one out
    size_t stage_bytes = 0;
    unsigned *hdone = nullptr;      // completion flags in coherent pinned memory
    unsigned done_seq = 0;          // the value the last flagged call wrote
    unsigned char *img = nullptr;   // prefill key-tile images, grown on demand
    size_t img_bytes = 0;
    float *ppartials = nullptr;     // prefill split-K partials, grown on demand
    size_t ppartials_bytes = 0;
    int *pcounters = nullptr;       // prefill split-K arrival counters
    size_t pcounters_n = 0;
};

namespace {

int herr(hipError_t e) { return e == hipSuccess ? TQ_HIP_OK : TQ_HIP_EHIP_BASE - (int)e; }

#define TQ_TRY(expr)                          \
    do {                                      \
        const hipError_t e_ = (expr);         \
        if (e_ != hipSuccess) return herr(e_); \
    } while (0)

hipStream_t pick(tq_hip_kv *kv, void *stream) {
    return stream ? static_cast<hipStream_t>(stream) : kv->stream;
}

// Work-groups the decode aims for on the 256-CU MI355X.  One sequence: four
// per CU, so that a 4k-token context is cut into 128-token splits over every
// CU.  A batch: two per CU, in one round of resident work-groups; each
// work-group's fixed cost (staging q, the wave merge, the split combine)
// outweighs the balance that shorter splits buy (64 ragged 512-8192 token
// sequences at the 8B shape: 117 us per step with one split per sequence and
// head, against 135-180 us at 1024-2048 work-groups).  Overridable for sweeps.
int decode_wg_target(int n_q) {
    static int v = [] {
        const char *s = getenv("TQ_HIP_DECODE_WG_TARGET");
        const int x = s ? atoi(s) : 0;
        return x > 0 ? x : 0;
    }();
    return v ? v : (n_q > 1 ? 512 : 1024);
}

// Fewest new tokens for which a prefill call uses the dense kernel.
constexpr int kPrefillDenseMin = 32;

// The dense MFMA prefill kernel (default) or, with TQ_HIP_PREFILL_DENSE=0,
// the decode kernel run once per token with causal lengths.
bool prefill_dense() {
    static bool v = [] {
        const char *s = getenv("TQ_HIP_PREFILL_DENSE");
        return !(s && s[0] == '0');
    }();
    return v;
}

int decode_max_splits() {
    static int v = [] {
        const char *s = getenv("TQ_HIP_DECODE_MAX_SPLITS");
        const int x = s ? atoi(s) : 0;
        return x > 0 ? x : 32;
    }();
    return v;
}

// Split the context of every query into n_splits ranges of split_tokens
// (a multiple of the kernel's sub-chunk) for n_q queries of up to max_len.
void plan_splits(const tq_hip_kv *kv, int n_q, int max_len, int *split_tokens, int *n_splits) {
    const int tsub = tq_decode_tsub(kv->desc.head_dim);
    const int chunks = std::max(1, (max_len + tsub - 1) / tsub);
    const long pairs = (long)n_q * kv->desc.n_kv_heads;
    const int cap = std::min(decode_max_splits(),
                             tq_decode_max_splits(kv->desc.head_dim, kv->desc.n_q_heads / kv->desc.n_kv_heads));
    long want = (decode_wg_target(n_q) + pairs - 1) / pairs;
    want = std::max(1L, std::min<long>(want, cap));
    want = std::min<long>(want, chunks);
    // a work-group stages at most tq_decode_max_split_tokens() page ids
    const int max_per = tq_decode_max_split_tokens() / tsub;
    want = std::max<long>(want, (chunks + max_per - 1) / max_per);
    const int per = (int)((chunks + want - 1) / want);
    *split_tokens = per * tsub;
    *n_splits = (chunks + per - 1) / per;
}

// Which decode kernel serves a call: the MFMA kernel (decode3.hip) wherever it
// covers the shape, else the VALU kernel (decode.hip).  TQ_HIP_DECODE_KERNEL=1
// forces the VALU kernel (for comparisons).
bool use_decode3(const tq_hip_kv *kv) {
    static int forced = [] {
        const char *s = getenv("TQ_HIP_DECODE_KERNEL");
        return s ? atoi(s) : 0;
    }();
    return forced != 1 && tq_decode3_supported(kv->desc.head_dim, kv->desc.n_q_heads / kv->desc.n_kv_heads);
}

// Longest split (tokens) the MFMA decode gives one work-group when the split
// count allows (TQ_HIP_DECODE_SPLIT_CAP, for sweeps); by default only the
// page-id staging limits it.
int decode3_split_cap() {
    static int v = [] {
        const char *s = getenv("TQ_HIP_DECODE_SPLIT_CAP");
        const int x = s ? atoi(s) : 0;
        return x > 0 ? x : tq_decode3_max_split_tokens();
    }();
    return v;
}

// Waves per work-group of the MFMA decode (TQ_HIP_DECODE_WAVES=4|8 forces it).
int decode3_waves_env() {
    static int v = [] {
        const char *s = getenv("TQ_HIP_DECODE_WAVES");
        const int x = s ? atoi(s) : 0;
        return (x == 4 || x == 8) ? x : 0;
    }();
    return v;
}

// MFMA decode: splits are whole units of 32*waves tokens (one tile per wave).
// Aim at decode_wg_target() work-groups, at most decode3_split_cap() tokens per
// split, and never more splits than the combine takes.
void plan_splits3(const tq_hip_kv *kv, int n_q, int max_len, int waves, int *split_tokens, int *n_splits) {
    const int unit = 32 * waves;
    const long units = std::max(1, (max_len + unit - 1) / unit);
    const long pairs = (long)n_q * kv->desc.n_kv_heads;
    const long cap = tq_decode3_max_splits();
    long want = (decode_wg_target(n_q) + pairs - 1) / pairs;
    want = std::max(1L, std::min(std::min(want, cap), units));
    long per = (units + want - 1) / want;
    per = std::min<long>(per, std::max(1, decode3_split_cap() / unit));
    per = std::max(per, (units + cap - 1) / cap);
    per = std::min<long>(per, tq_decode3_max_split_tokens() / unit);
    *split_tokens = (int)(per * unit);
    *n_splits = (int)((units + per - 1) / per);
}

// Longest context one decode call serves for this cache's shape.
long max_context(const tq_hip_kv *kv) {
    const int g = kv->desc.n_q_heads / kv->desc.n_kv_heads;
    return (long)tq_decode_max_splits(kv->desc.head_dim, g) * tq_decode_max_split_tokens();
}

int ensure_partials(tq_hip_kv *kv, size_t bytes) {
    if (bytes <= kv->partials_bytes) return TQ_HIP_OK;
    if (kv->partials) {
        TQ_TRY(hipDeviceSynchronize());
        TQ_TRY(hipFree(kv->partials));
        kv->partials = nullptr;
        kv->partials_bytes = 0;
    }
    if (hipMalloc(&kv->partials, bytes) != hipSuccess) {
        kv->partials = nullptr;
        return TQ_HIP_ENOMEM;
    }
    kv->partials_bytes = bytes;
    return TQ_HIP_OK;
}

// Counters are zeroed once when allocated, on the stream of the launch that
// will use them and synchronously (never inside a captured graph: warm up
// first); the decode kernel's combining work-group puts each back to 0.
int ensure_counters(tq_hip_kv *kv, size_t n, hipStream_t s) {
    if (n <= kv->counters_n) return TQ_HIP_OK;
    if (kv->counters) {
        TQ_TRY(hipDeviceSynchronize());
        TQ_TRY(hipFree(kv->counters));
        kv->counters = nullptr;
        kv->counters_n = 0;
    }
    if (hipMalloc(&kv->counters, n * sizeof(int)) != hipSuccess) {
        kv->counters = nullptr;
        return TQ_HIP_ENOMEM;
    }
    TQ_TRY(hipMemsetAsync(kv->counters, 0, n * sizeof(int), s));
    TQ_TRY(hipStreamSynchronize(s));
    kv->counters_n = n;
    return TQ_HIP_OK;
}

int ensure_img(tq_hip_kv *kv, size_t bytes) {
    if (bytes <= kv->img_bytes) return TQ_HIP_OK;
    if (kv->img) {
        TQ_TRY(hipDeviceSynchronize());
        TQ_TRY(hipFree(kv->img));
        kv->img = nullptr;
        kv->img_bytes = 0;
    }
    if (hipMalloc(&kv->img, bytes) != hipSuccess) {
        kv->img = nullptr;
        return TQ_HIP_ENOMEM;
    }
    kv->img_bytes = bytes;
    return TQ_HIP_OK;
}

// Prefill split-K scratch: partials (grown), counters (grown, zeroed once; the
// kernel's merging work-group puts each back to 0).
int ensure_prefill_scratch(tq_hip_kv *kv, size_t pbytes, size_t cn, hipStream_t s) {
    if (pbytes > kv->ppartials_bytes) {
        TQ_TRY(hipDeviceSynchronize());
        if (kv->ppartials) TQ_TRY(hipFree(kv->ppartials));
        kv->ppartials = nullptr;
        kv->ppartials_bytes = 0;
        if (hipMalloc(&kv->ppartials, pbytes) != hipSuccess) {
            kv->ppartials = nullptr;
            return TQ_HIP_ENOMEM;
        }
        kv->ppartials_bytes = pbytes;
    }
    if (cn > kv->pcounters_n) {
        TQ_TRY(hipDeviceSynchronize());
        if (kv->pcounters) TQ_TRY(hipFree(kv->pcounters));
        kv->pcounters = nullptr;
        kv->pcounters_n = 0;
        if (hipMalloc(&kv->pcounters, cn * sizeof(int)) != hipSuccess) {
            kv->pcounters = nullptr;
            return TQ_HIP_ENOMEM;
        }
        TQ_TRY(hipMemsetAsync(kv->pcounters, 0, cn * sizeof(int), s));
        TQ_TRY(hipStreamSynchronize(s));
        kv->pcounters_n = cn;
    }
    return TQ_HIP_OK;
}

int ensure_stage(tq_hip_kv *kv, size_t bytes) {
    if (bytes <= kv->stage_bytes) return TQ_HIP_OK;
    TQ_TRY(hipStreamSynchronize(kv->stream));
    if (kv->stage) TQ_TRY(hipFree(kv->stage));
    if (kv->hstage) TQ_TRY(hipHostFree(kv->hstage));
    kv->stage = nullptr;
    kv->hstage = nullptr;
    kv->stage_bytes = 0;
    if (hipMalloc(&kv->stage, bytes) != hipSuccess) {
        kv->stage = nullptr;
        return TQ_HIP_ENOMEM;
    }
    if (hipHostMalloc(&kv->hstage, bytes, hipHostMallocDefault) != hipSuccess) {
        kv->hstage = nullptr;
        (void)hipFree(kv->stage);
        kv->stage = nullptr;
        return TQ_HIP_ENOMEM;
    }
    kv->stage_bytes = bytes;
    return TQ_HIP_OK;
}

struct Stage {
    size_t used = 0;
    size_t take(size_t bytes) {
        const size_t at = used;
        used += (bytes + 255) & ~(size_t)255;
        return at;
    }
};

// The synchronous entry points: host inputs are packed into the pinned mirror.
// Up to kDirectIn bytes of them the decode kernel reads there itself, over the
// bus (its L2 serves the work-groups that share a line); larger inputs are
// moved to the device staging area first by one small copy kernel (a kernel
// launch costs less than a copy-engine transfer of a few KB: 12.8 against
// 8.4 + ~4 us per round trip measured on MI355X, where hipMemcpyAsync hands
// the copy to another engine and the next launch waits on it).  Outputs of up
// to kDirectOut bytes are written by the kernel itself into the pinned mirror,
// which the device sees at the same address; larger outputs come back with one
// copy.  The MFMA decode then raises one completion flag per (query, kv head)
// in coherent pinned memory after its rows are acknowledged at system scope,
// and the host spins on those flags rather than on the stream: 6.1 against
// 9.5 us for an empty kernel's round trip on MI355X.
constexpr size_t kDirectIn = 64u << 10;
constexpr size_t kDirectOut = 64u << 10;
constexpr int kDoneFlags = 4096;

// Completion flags of one synchronous call: armed by decode_common when the
// kernel it launches will raise them.
struct DoneFlags {
    unsigned *flags = nullptr;
    unsigned seq = 0;
    int count = 0;
    bool armed = false;
};

int ensure_done(tq_hip_kv *kv) {
    if (kv->hdone) return TQ_HIP_OK;
    void *p = nullptr;
    if (hipHostMalloc(&p, kDoneFlags * sizeof(unsigned), hipHostMallocCoherent) != hipSuccess) return TQ_HIP_ENOMEM;
    memset(p, 0, kDoneFlags * sizeof(unsigned));
    kv->hdone = static_cast<unsigned *>(p);
    kv->done_seq = 0;
    return TQ_HIP_OK;
}

// Flags for the next synchronous call on kv (never the value 0 they start at).
DoneFlags next_done(tq_hip_kv *kv) {
    DoneFlags d;
    if (ensure_done(kv) != TQ_HIP_OK) return d;
    if (++kv->done_seq == 0) kv->done_seq = 1;
    d.flags = kv->hdone;
    d.seq = kv->done_seq;
    return d;
}

// Until every armed flag holds the call's value, or the stream has drained
// (flags a query never raises, e.g. one with nothing to attend) or failed.
// The stream is asked only once the flags are late (kLateUs after the wait
// began, then every kLateUs): hipStreamQuery costs about as much as the call
// it would check, and asked every few hundred spins it landed inside calls
// whose flags come 6-9 us after launch (store_kv_device 9 -> 20 us).
constexpr double kLateUs = 25.0;
double now_us() {
    timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return (double)t.tv_sec * 1e6 + (double)t.tv_nsec * 1e-3;
}
int wait_done(tq_hip_kv *kv, const DoneFlags &d) {
    double ask_at = now_us() + kLateUs;
    for (unsigned it = 1;; it++) {
        bool all = true;
        for (int i = 0; i < d.count && all; i++) all = __atomic_load_n(d.flags + i, __ATOMIC_ACQUIRE) == d.seq;
        if (all) return TQ_HIP_OK;
        __builtin_ia32_pause();   // a spin-wait hint to the core, not a yield
        if ((it & 63u) == 0) {
            const double t = now_us();
            if (t >= ask_at) {
                const hipError_t e = hipStreamQuery(kv->stream);
                if (e != hipErrorNotReady) return herr(e);
                ask_at = t + kLateUs;
            }
        }
    }
}

__global__ __launch_bounds__(256) void stage_in_kernel(const uint4 *src, uint4 *dst, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) dst[i] = src[i];
}

void pack(tq_hip_kv *kv, size_t off, const void *src, size_t bytes) {
    if (src) memcpy(kv->hstage + off, src, bytes);
}
// bytes: a multiple of 16 (Stage rounds every piece to 256)
int copy_in(tq_hip_kv *kv, size_t bytes) {
    const size_t n = bytes / 16;
    const unsigned blocks = (unsigned)std::min<size_t>(64, (n + 255) / 256);
    hipLaunchKernelGGL(stage_in_kernel, dim3(blocks), dim3(256), 0, kv->stream,
                       reinterpret_cast<const uint4 *>(kv->hstage), reinterpret_cast<uint4 *>(kv->stage), n);
    return herr(hipGetLastError());
}
// Where the kernel writes an output of `bytes` at staging offset `off`.
float *out_slot(tq_hip_kv *kv, size_t off, size_t bytes) {
    return reinterpret_cast<float *>((bytes <= kDirectOut ? kv->hstage : kv->stage) + off);
}
int copy_out_sync(tq_hip_kv *kv, void *dst, size_t off, size_t bytes, const DoneFlags *done = nullptr) {
    if (bytes > kDirectOut)
        TQ_TRY(hipMemcpyAsync(kv->hstage + off, kv->stage + off, bytes, hipMemcpyDeviceToHost, kv->stream));
    if (bytes <= kDirectOut && done && done->armed) {
        const int rc = wait_done(kv, *done);
        if (rc != TQ_HIP_OK) return rc;
    } else {
        TQ_TRY(hipStreamSynchronize(kv->stream));
    }
    memcpy(dst, kv->hstage + off, bytes);
    return TQ_HIP_OK;
}
// The inputs the kernel reads: the pinned mirror itself when they are small
// (no copy kernel), else their device copy, made here.
int inputs_at(tq_hip_kv *kv, size_t in_bytes, bool may_read_host, unsigned char **base) {
    if (may_read_host && in_bytes <= kDirectIn) {
        *base = kv->hstage;
        return TQ_HIP_OK;
    }
    *base = kv->stage;
    return copy_in(kv, in_bytes);
}

int capacity_of(const tq_hip_kv *kv, int seq);

// A sequence whose mapped logical pages 0..n-1 are physical first..first+n-1.
void seq_contig(const tq_hip_kv *kv, int seq, int *first, int *n) {
    const int32_t *row = kv->h_page_table.data() + (size_t)seq * kv->desc.max_pages_per_seq;
    *first = row[0];
    *n = 0;
    if (row[0] < 0) return;
    while (*n < kv->desc.max_pages_per_seq && row[*n] == row[0] + *n) (*n)++;
}

// Split-K scratch a call brings instead of the cache's own (grown) buffers.
struct CallScratch {
    float *partials;
    size_t partial_bytes;
    int *counters;         // zero between launches
    size_t counter_ints;
};

// contig_seq: the one sequence every query of this call reads, or -1.
// q_norm non-null: q (and the new K) are raw projections, RMSNorm'd in the
// kernel with q_norm / k_norm and eps (MFMA kernel only).
// scratch non-null: the split-K partials and counters come from it (a call
// that needs more returns TQ_HIP_ESCRATCH) and nothing is allocated.
int decode_common(tq_hip_kv *kv, int n_q, const int32_t *d_seq, const int32_t *d_len, int len_plus,
                  int seq_const, int seq_stride, int pos0, int max_len, const float *d_q, const float *d_cos,
                  const float *d_sin, const float *d_k, const float *d_v, float *d_out,
                  hipStream_t s, int contig_seq, const float *q_norm = nullptr,
                  const float *k_norm = nullptr, float rms_eps = 0.0f, const CallScratch *scratch = nullptr,
                  DoneFlags *done = nullptr) {
    if (n_q <= 0) return TQ_HIP_OK;
    // queries and kv heads are grid dimensions y/z (at most 65535 each)
    if (n_q > 65535 || kv->desc.n_kv_heads > 65535) return TQ_HIP_EINVAL;
    if (max_len <= 0 || !d_q || !d_out) return TQ_HIP_EINVAL;
    // contexts longer than n_splits * split_tokens allows are not served
    if ((long)max_len > max_context(kv)) return TQ_HIP_EINVAL;
    if ((d_cos == nullptr) != (d_sin == nullptr)) return TQ_HIP_EINVAL;
    const tq_hip_kv_desc &D = kv->desc;
    TqDecodeArgs a{};
    a.view = kv->view;
    a.seq_of = d_seq;
    a.len_of = d_len;
    a.len_plus = len_plus;
    a.seq_const = seq_const;
    a.seq_stride = seq_stride;
    a.pos0 = pos0;
    a.q = d_q;
    a.cos_t = d_cos;
    a.sin_t = d_sin;
    a.k_new = d_k;
    a.v_new = d_v;
    a.q_norm = q_norm;
    a.k_norm = k_norm;
    a.rms_eps = rms_eps;
    a.out = d_out;
    a.n_q = n_q;
    a.n_q_heads = D.n_q_heads;
    a.n_kv_heads = D.n_kv_heads;
    a.head_dim = D.head_dim;
    a.scale = 1.0f / sqrtf((float)D.head_dim);  // model/attention_layer.c:131
    a.contig_first = -1;
    a.contig_pages = 0;
    if (contig_seq >= 0) {
        int first, n;
        seq_contig(kv, contig_seq, &first, &n);
        // the whole mapped range must be one run for the kernel to skip the table
        if (n > 0 && n * TQ_HIP_PAGE_TOKENS >= capacity_of(kv, contig_seq)) {
            a.contig_first = first;
            a.contig_pages = n;
        }
    }
    // the MFMA kernel copies its inputs with 16-byte loads
    const bool aligned = (((uintptr_t)d_q | (uintptr_t)d_cos | (uintptr_t)d_sin | (uintptr_t)d_k | (uintptr_t)d_v) &
                          15) == 0;
    const bool v3 = aligned && use_decode3(kv);
    if (q_norm) {
        // the norm is fused into the MFMA kernel only; it stages 16-byte pieces
        if (((uintptr_t)q_norm | (uintptr_t)k_norm) & 15) return TQ_HIP_EINVAL;
        if (!v3) return TQ_HIP_ETYPE;
    }
    // four waves per work-group: for a single 4k-token sequence at the 8B
    // shape this spreads one 32-key tile per wave over all 256 CUs, which beats
    // eight waves on half of them (8.7 against 9.1 us per step).  A batch at
    // G <= 4 takes eight: two resident work-groups per CU then stream 16 tiles
    // at once (the 64-sequence batch: 117 against 129 us); at G = 8 four waves
    // stay ahead (234 against 240 us at 16 x 32k tokens).
    const int g = D.n_q_heads / D.n_kv_heads;
    int waves = n_q > 1 && g <= 4 ? 8 : 4;
    // one query over at most 256 keys: eight waves of one 32-key tile each in
    // one work-group per kv head, with no split-K combine (its store, counter
    // and pull cost more than the tiles: 8B shape at 256 keys 7.1 -> 6.2 us,
    // 8q/2kv/hd64 6.6 -> 5.3 us; from 384 keys on the splits win)
    if (n_q == 1 && max_len <= 8 * 32) waves = 8;
    if (decode3_waves_env()) waves = decode3_waves_env();
    if (v3)
        plan_splits3(kv, n_q, max_len, waves, &a.split_tokens, &a.n_splits);
    else
        plan_splits(kv, n_q, max_len, &a.split_tokens, &a.n_splits);
    if (a.n_splits > 1) {
        const size_t row = v3 ? (size_t)tq_decode3_partial_floats(D.head_dim, g) : (size_t)g * (D.head_dim + 2);
        const size_t bytes = (size_t)n_q * D.n_kv_heads * a.n_splits * row * sizeof(float);
        const size_t n_counters = (size_t)n_q * D.n_kv_heads * TQ_DECODE_COUNTER_STRIDE;
        if (scratch) {
            if (bytes > scratch->partial_bytes || n_counters > scratch->counter_ints) return TQ_HIP_ESCRATCH;
            a.partials = scratch->partials;
            a.counters = scratch->counters;
        } else {
            int rc = ensure_partials(kv, bytes);
            if (rc == TQ_HIP_OK) rc = ensure_counters(kv, n_counters, s);
            if (rc != TQ_HIP_OK) return rc;
            a.partials = kv->partials;
            a.counters = kv->counters;
        }
    }
    if (v3 && done && done->flags && (long)n_q * D.n_kv_heads <= kDoneFlags) {
        a.done = done->flags;
        a.done_seq = done->seq;
        done->count = n_q * D.n_kv_heads;
        done->armed = true;
    }
    return herr(v3 ? tq_launch_decode3(a, waves, s) : tq_launch_decode(a, s));
}

// ---- the allocation-free decode step's scratch ----------------------------
// One fixed array per GPU, held until the process ends: [arrival counters |
// split-K partial rows].  Host code never passes `scratch` itself (its name is
// a host-side stand-in); it uses the device address hipGetSymbolAddress
// returned for the current device.
constexpr size_t kNoAllocCounterBytes = 256u << 10;   // 1024 (query, kv head) pairs x 256 B
static_assert(TQ_HIP_NOALLOC_SCRATCH_BYTES % 256 == 0 && TQ_HIP_NOALLOC_SCRATCH_BYTES > kNoAllocCounterBytes,
              "scratch layout");
static __device__ __align__(256) unsigned char scratch[TQ_HIP_NOALLOC_SCRATCH_BYTES];

__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t *p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) p[i] = 0u;
}

constexpr int kMaxDevices = 64;
struct NoAllocDevice {
    std::once_flag once;
    unsigned char *ptr = nullptr;   // scratch on this device
    int rc = TQ_HIP_OK;
};
NoAllocDevice g_noalloc[kMaxDevices];

// Once per device, with that device current: look up the array's device
// address and clear its counters (a fill kernel, then a wait: not inside a
// graph capture).  The decode kernel's combining work-group puts every
// counter it used back to 0, so they stay zero between calls.
int noalloc_setup(int device) {
    if (device < 0 || device >= kMaxDevices) return TQ_HIP_ENODEV;
    NoAllocDevice &d = g_noalloc[device];
    std::call_once(d.once, [&d] {
        void *p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e == hipSuccess) {
            hipLaunchKernelGGL(zero_words_kernel, dim3(64), dim3(256), 0, nullptr, static_cast<uint32_t *>(p),
                               kNoAllocCounterBytes / 4);
            e = hipGetLastError();
        }
        if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
        d.rc = herr(e);
        if (e == hipSuccess) d.ptr = static_cast<unsigned char *>(p);
    });
    return d.rc;
}

bool seq_ok(const tq_hip_kv *kv, int seq) { return kv && seq >= 0 && seq < kv->desc.max_seqs; }

int capacity_of(const tq_hip_kv *kv, int seq) {
    int mapped = 0;
    const int32_t *row = kv->h_page_table.data() + (size_t)seq * kv->desc.max_pages_per_seq;
    while (mapped < kv->desc.max_pages_per_seq && row[mapped] >= 0) mapped++;
    return mapped * TQ_HIP_PAGE_TOKENS;
}

}  // namespace

extern "C" {

int tq_hip_init(int device) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return TQ_HIP_ENODEV;
    if (device < 0 || device >= n) return TQ_HIP_EINVAL;
    TQ_TRY(hipSetDevice(device));
    hipDeviceProp_t p;
    TQ_TRY(hipGetDeviceProperties(&p, device));
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0) return TQ_HIP_ENODEV;
    // the allocation-free entry point's scratch is set up here, once per
    // device; a failure is kept for tq_hip_decode_step_noalloc to return and
    // does not fail the init of callers that never use it
    (void)noalloc_setup(device);
    return TQ_HIP_OK;
}

const char *tq_hip_strerror(int code) {
    switch (code) {
        case TQ_HIP_OK: return "ok";
        case TQ_HIP_EINVAL: return "argument out of range";
        case TQ_HIP_ENOMEM: return "out of memory";
        case TQ_HIP_ETYPE: return "unsupported head_dim or group size";
        case TQ_HIP_ENODEV: return "no gfx950 device";
        case TQ_HIP_ENOTREADY: return "position has no mapped page";
        case TQ_HIP_ESCRATCH: return "call needs more split-K scratch than the allocation-free entry point holds";
        default: break;
    }
    if (code <= TQ_HIP_EHIP_BASE) return hipGetErrorString((hipError_t)(TQ_HIP_EHIP_BASE - code));
    return "unknown error";
}

int tq_hip_device_arch(char *buf, size_t len) {
    if (!buf || len == 0) return TQ_HIP_EINVAL;
    int dev = 0;
    TQ_TRY(hipGetDevice(&dev));
    hipDeviceProp_t p;
    TQ_TRY(hipGetDeviceProperties(&p, dev));
    strncpy(buf, p.gcnArchName, len - 1);
    buf[len - 1] = 0;
    return TQ_HIP_OK;
}

int tq_hip_malloc(void **ptr, size_t bytes) {
    if (!ptr) return TQ_HIP_EINVAL;
    *ptr = nullptr;
    if (bytes == 0) return TQ_HIP_OK;
    const hipError_t e = hipMalloc(ptr, bytes);
    if (e == hipErrorOutOfMemory) return TQ_HIP_ENOMEM;
    return herr(e);
}

int tq_hip_free(void *ptr) { return ptr ? herr(hipFree(ptr)) : TQ_HIP_OK; }

int tq_hip_memcpy_h2d(void *dst, const void *src, size_t bytes, void *stream) {
    if (bytes == 0) return TQ_HIP_OK;
    if (!dst || !src) return TQ_HIP_EINVAL;
    if (!stream) return herr(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return herr(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream));
}

int tq_hip_memcpy_d2h(void *dst, const void *src, size_t bytes, void *stream) {
    if (bytes == 0) return TQ_HIP_OK;
    if (!dst || !src) return TQ_HIP_EINVAL;
    if (!stream) return herr(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return herr(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream));
}

int tq_hip_memcpy_d2d(void *dst, const void *src, size_t bytes, void *stream) {
    if (bytes == 0) return TQ_HIP_OK;
    if (!dst || !src) return TQ_HIP_EINVAL;
    if (!stream) return herr(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice));
    return herr(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream));
}

int tq_hip_stream_synchronize(void *stream) { return herr(hipStreamSynchronize((hipStream_t)stream)); }
int tq_hip_device_synchronize(void) { return herr(hipDeviceSynchronize()); }

// ---- kernel-level ops ------------------------------------------------------

int tq_hip_quantize_row_q8(const float *x, block_q8 *out, int n, void *stream) {
    if (n < 0 || (n > 0 && (!x || !out))) return TQ_HIP_EINVAL;
    if (((uintptr_t)x | (uintptr_t)out) & 3) return TQ_HIP_EINVAL;   // the kernels store dwords
    return herr(tq_launch_quantize(x, out, n, (hipStream_t)stream));
}

int tq_hip_rope_apply(float *x, int n_heads, int head_dim, const float *cos_t, const float *sin_t,
                      void *stream) {
    if (n_heads < 0 || head_dim < 2 || (head_dim & 1) || !x || !cos_t || !sin_t) return TQ_HIP_EINVAL;
    return herr(tq_launch_rope(x, n_heads, head_dim, cos_t, sin_t, (hipStream_t)stream));
}

int tq_hip_attn_scores_q8(const block_q8 *q, int g, const block_q8 *k, int n, int nb, float scale,
                          float *scores, size_t stride, void *stream) {
    if (g <= 0 || n < 0 || nb <= 0 || stride < (size_t)n || !q || (n > 0 && (!k || !scores)))
        return TQ_HIP_EINVAL;
    return herr(tq_launch_scores(q, g, k, n, nb, scale, scores, stride, (hipStream_t)stream));
}

int tq_hip_attn_accum_q8(const float *w, size_t w_stride, int g, const block_q8 *v, int n, int nb,
                         float *out, size_t out_stride, void *stream) {
    if (g <= 0 || n < 0 || nb <= 0 || out_stride < (size_t)nb * QK || w_stride < (size_t)n || !out ||
        (n > 0 && (!w || !v)))
        return TQ_HIP_EINVAL;
    return herr(tq_launch_accum(w, w_stride, g, v, n, nb, out, out_stride, (hipStream_t)stream));
}

int tq_hip_rmsnorm_rows(const float *x, const float *weight, float *out, int n_rows, int n, float eps,
                        void *stream) {
    if (n_rows < 0 || n <= 0 || n > 8191 || (n_rows > 0 && (!x || !weight || !out))) return TQ_HIP_EINVAL;
    return herr(tq_launch_rmsnorm_rows(x, weight, out, n_rows, n, eps, (hipStream_t)stream));
}

int tq_hip_softmax(float *x, int n, int rows, size_t stride, void *stream) {
    if (n < 0 || rows < 0 || (rows > 1 && stride < (size_t)n) || (n > 0 && rows > 0 && !x))
        return TQ_HIP_EINVAL;
    return herr(tq_launch_softmax(x, n, rows, stride, (hipStream_t)stream));
}

int tq_hip_attention_head_q8(const float *q, block_q8 *q_q8, const block_q8 *k_cache,
                             const block_q8 *v_cache, int n, int head_dim, float *scores, float *out,
                             void *stream) {
    if (head_dim <= 0 || head_dim % QK || n <= 0 || !q || !q_q8 || !k_cache || !v_cache || !scores || !out)
        return TQ_HIP_EINVAL;
    const hipStream_t s = (hipStream_t)stream;
    const int nb = head_dim / QK;
    const float scale = 1.0f / sqrtf((float)head_dim);  // model/attn_q8.c:83
    TQ_TRY(tq_launch_quantize(q, q_q8, head_dim, s));
    TQ_TRY(tq_launch_scores(q_q8, 1, k_cache, n, nb, scale, scores, (size_t)n, s));
    TQ_TRY(tq_launch_softmax(scores, n, 1, (size_t)n, s));
    return herr(tq_launch_accum(scores, (size_t)n, 1, v_cache, n, nb, out, (size_t)head_dim, s));
}

// ---- paged cache -------------------------------------------------------------

int tq_hip_kv_create(tq_hip_kv **out, const tq_hip_kv_desc *desc) {
    if (!out) return TQ_HIP_EINVAL;
    *out = nullptr;
    if (!desc) return TQ_HIP_EINVAL;
    const tq_hip_kv_desc D = *desc;
    // model/attention_layer.c:11,16-17 (tq_attn_validate -8, -5, -6)
    if (D.n_q_heads <= 0 || D.n_kv_heads <= 0 || D.head_dim <= 0) return TQ_HIP_EINVAL;
    if (D.n_q_heads % D.n_kv_heads != 0 || D.head_dim % QK != 0) return TQ_HIP_EINVAL;
    if (D.n_pages <= 0 || D.max_seqs <= 0 || D.max_pages_per_seq <= 0) return TQ_HIP_EINVAL;
    if (!tq_decode_supported(D.head_dim, D.n_q_heads / D.n_kv_heads)) return TQ_HIP_ETYPE;

    tq_hip_kv *kv = new (std::nothrow) tq_hip_kv();
    if (!kv) return TQ_HIP_ENOMEM;
    kv->desc = D;
    int rc = herr(hipGetDevice(&kv->device));
    const int nb = D.head_dim / QK;
    tq::PagedView &v = kv->view;
    v.nb = nb;
    v.row_bytes = (size_t)nb * sizeof(block_q8);
    v.kv_chunk = (size_t)TQ_HIP_PAGE_TOKENS * v.row_bytes;
    v.head_run = 2 * v.kv_chunk;
    v.page_bytes = (size_t)D.n_kv_heads * v.head_run;
    v.n_pages = D.n_pages;
    v.max_seqs = D.max_seqs;
    v.max_pages = D.max_pages_per_seq;
    v.n_kv_heads = D.n_kv_heads;
    kv->pool_bytes = (size_t)D.n_pages * v.page_bytes;
    const size_t pt_entries = (size_t)D.max_seqs * D.max_pages_per_seq;
    try {
        kv->h_page_table.assign(pt_entries, -1);
    } catch (...) {
        delete kv;
        return TQ_HIP_ENOMEM;
    }
    if (rc == TQ_HIP_OK) rc = herr(hipStreamCreateWithFlags(&kv->stream, hipStreamNonBlocking));
    if (rc == TQ_HIP_OK && hipMalloc(&kv->pool, kv->pool_bytes) != hipSuccess) {
        kv->pool = nullptr;
        rc = TQ_HIP_ENOMEM;
    }
    if (rc == TQ_HIP_OK && hipMalloc(&kv->d_page_table, pt_entries * sizeof(int32_t)) != hipSuccess) {
        kv->d_page_table = nullptr;
        rc = TQ_HIP_ENOMEM;
    }
    if (rc == TQ_HIP_OK) rc = herr(hipMemsetAsync(kv->pool, 0, kv->pool_bytes, kv->stream));
    if (rc == TQ_HIP_OK)
        rc = herr(hipMemsetAsync(kv->d_page_table, 0xFF, pt_entries * sizeof(int32_t), kv->stream));
    if (rc == TQ_HIP_OK) rc = herr(hipStreamSynchronize(kv->stream));
    if (rc != TQ_HIP_OK) {
        tq_hip_kv_destroy(kv);
        return rc;
    }
    v.pool = kv->pool;
    v.page_table = kv->d_page_table;
    *out = kv;
    return TQ_HIP_OK;
}

void tq_hip_kv_destroy(tq_hip_kv *kv) {
    if (!kv) return;
    if (kv->stream) (void)hipStreamSynchronize(kv->stream);
    if (kv->pool) (void)hipFree(kv->pool);
    if (kv->d_page_table) (void)hipFree(kv->d_page_table);
    if (kv->partials) (void)hipFree(kv->partials);
    if (kv->counters) (void)hipFree(kv->counters);
    if (kv->stage) (void)hipFree(kv->stage);
    if (kv->hstage) (void)hipHostFree(kv->hstage);
    if (kv->hdone) (void)hipHostFree(kv->hdone);
    if (kv->img) (void)hipFree(kv->img);
    if (kv->ppartials) (void)hipFree(kv->ppartials);
    if (kv->pcounters) (void)hipFree(kv->pcounters);
    if (kv->stream) (void)hipStreamDestroy(kv->stream);
    delete kv;
}

int tq_hip_kv_set_pages(tq_hip_kv *kv, int seq, const int32_t *pages, int n_pages) {
    if (!seq_ok(kv, seq) || n_pages < 0 || n_pages > kv->desc.max_pages_per_seq) return TQ_HIP_EINVAL;
    if (n_pages > 0 && !pages) return TQ_HIP_EINVAL;
    for (int i = 0; i < n_pages; i++)
        if (pages[i] < -1 || pages[i] >= kv->desc.n_pages) return TQ_HIP_EINVAL;
    int32_t *row = kv->h_page_table.data() + (size_t)seq * kv->desc.max_pages_per_seq;
    for (int i = 0; i < kv->desc.max_pages_per_seq; i++) row[i] = i < n_pages ? pages[i] : -1;
    TQ_TRY(hipMemcpyAsync(kv->d_page_table + (size_t)seq * kv->desc.max_pages_per_seq, row,
                          (size_t)kv->desc.max_pages_per_seq * sizeof(int32_t), hipMemcpyHostToDevice,
                          kv->stream));
    return herr(hipStreamSynchronize(kv->stream));
}

int tq_hip_kv_capacity(const tq_hip_kv *kv, int seq) {
    if (!seq_ok(kv, seq)) return TQ_HIP_EINVAL;
    return capacity_of(kv, seq);
}

int tq_hip_kv_get_desc(const tq_hip_kv *kv, tq_hip_kv_desc *desc) {
    if (!kv || !desc) return TQ_HIP_EINVAL;
    *desc = kv->desc;
    return TQ_HIP_OK;
}

void *tq_hip_kv_stream(tq_hip_kv *kv) { return kv ? (void *)kv->stream : nullptr; }

int tq_hip_kv_pool(tq_hip_kv *kv, void **base, size_t *bytes, int32_t **page_table) {
    if (!kv) return TQ_HIP_EINVAL;
    if (base) *base = kv->pool;
    if (bytes) *bytes = kv->pool_bytes;
    if (page_table) *page_table = kv->d_page_table;
    return TQ_HIP_OK;
}

// Copy rows [pos0, pos0+n) page by page; `to_device` patches rows into
// the pages (read-modify-write of each touched page run).
static int kv_rows(tq_hip_kv *kv, int seq, int pos0, int n, block_q8 *k, block_q8 *v, bool to_device) {
    if (!seq_ok(kv, seq) || pos0 < 0 || n < 0) return TQ_HIP_EINVAL;
    if (n == 0) return TQ_HIP_OK;
    if (pos0 + n > capacity_of(kv, seq)) return TQ_HIP_EINVAL;
    const tq::PagedView &V = kv->view;
    const int nkv = kv->desc.n_kv_heads, nb = V.nb;
    std::vector<unsigned char> run(V.head_run);
    const int32_t *pt = kv->h_page_table.data() + (size_t)seq * kv->desc.max_pages_per_seq;
    for (int lp = pos0 / TQ_HIP_PAGE_TOKENS; lp * TQ_HIP_PAGE_TOKENS < pos0 + n; lp++) {
        const int phys = pt[lp];
        for (int h = 0; h < nkv; h++) {
            unsigned char *dev = kv->pool + (size_t)phys * V.page_bytes + (size_t)h * V.head_run;
            TQ_TRY(hipMemcpy(run.data(), dev, V.head_run, hipMemcpyDeviceToHost));
            for (int r = 0; r < TQ_HIP_PAGE_TOKENS; r++) {
                const int pos = lp * TQ_HIP_PAGE_TOKENS + r;
                if (pos < pos0 || pos >= pos0 + n) continue;
                const size_t hoff = ((size_t)h * n + (pos - pos0)) * nb;
                unsigned char *kr = run.data() + (size_t)r * V.row_bytes;
                unsigned char *vr = kr + V.kv_chunk;
                if (to_device) {
                    if (k) memcpy(kr, k + hoff, V.row_bytes);
                    if (v) memcpy(vr, v + hoff, V.row_bytes);
                } else {
                    if (k) memcpy(k + hoff, kr, V.row_bytes);
                    if (v) memcpy(v + hoff, vr, V.row_bytes);
                }
            }
            if (to_device) TQ_TRY(hipMemcpy(dev, run.data(), V.head_run, hipMemcpyHostToDevice));
        }
    }
    return TQ_HIP_OK;
}

int tq_hip_kv_write(tq_hip_kv *kv, int seq, int pos0, int n, const block_q8 *k, const block_q8 *v) {
    if (kv) TQ_TRY(hipStreamSynchronize(kv->stream));
    return kv_rows(kv, seq, pos0, n, const_cast<block_q8 *>(k), const_cast<block_q8 *>(v), true);
}

int tq_hip_kv_read(tq_hip_kv *kv, int seq, int pos0, int n, block_q8 *k, block_q8 *v) {
    if (kv) TQ_TRY(hipStreamSynchronize(kv->stream));
    return kv_rows(kv, seq, pos0, n, k, v, false);
}

// ---- append --------------------------------------------------------------------

int tq_hip_kv_append_async(tq_hip_kv *kv, int n_rows, const int32_t *d_seq, const int32_t *d_pos,
                           const float *d_k, const float *d_v, const float *d_cos, const float *d_sin,
                           void *stream) {
    if (!kv || n_rows < 0) return TQ_HIP_EINVAL;
    if (n_rows == 0) return TQ_HIP_OK;
    if (!d_seq || !d_pos || !d_k || !d_v || ((d_cos == nullptr) != (d_sin == nullptr))) return TQ_HIP_EINVAL;
    return herr(tq_launch_append(kv->view, n_rows, d_seq, d_pos, 0, 0, d_k, d_v, d_cos, d_sin,
                                 kv->desc.head_dim, pick(kv, stream)));
}

int tq_hip_kv_append(tq_hip_kv *kv, int seq, int pos, const float *k, const float *v, const float *cos_t,
                     const float *sin_t) {
    if (!seq_ok(kv, seq) || !k || !v || ((cos_t == nullptr) != (sin_t == nullptr))) return TQ_HIP_EINVAL;
    if (pos < 0 || pos >= capacity_of(kv, seq)) return TQ_HIP_EINVAL;  // model/attention_layer.c:68,172
    const tq_hip_kv_desc &D = kv->desc;
    const size_t kvb = (size_t)D.n_kv_heads * D.head_dim * sizeof(float);
    const size_t tb = (size_t)(D.head_dim / 2) * sizeof(float);
    Stage st;
    const size_t ok_ = st.take(kvb), ov = st.take(kvb), oc = st.take(tb), os = st.take(tb);
    int rc = ensure_stage(kv, st.used);
    if (rc != TQ_HIP_OK) return rc;
    const hipStream_t s = kv->stream;
    unsigned char *S = nullptr;
    pack(kv, ok_, k, kvb);
    pack(kv, ov, v, kvb);
    pack(kv, oc, cos_t, tb);
    pack(kv, os, sin_t, tb);
    rc = inputs_at(kv, st.used, true, &S);
    if (rc != TQ_HIP_OK) return rc;
    // the host waits on the work-groups' completion flags (raised once the
    // inputs are read and the rows stored), not on the stream: later work on
    // kv's stream is ordered after the append either way
    DoneFlags d = next_done(kv);
    const bool flags = d.flags && D.n_kv_heads <= kDoneFlags;
    TQ_TRY(tq_launch_append(kv->view, 1, nullptr, nullptr, seq, pos, (const float *)(S + ok_),
                            (const float *)(S + ov), cos_t ? (const float *)(S + oc) : nullptr,
                            cos_t ? (const float *)(S + os) : nullptr, D.head_dim, s, flags ? d.flags : nullptr,
                            d.seq));
    if (!flags) return herr(hipStreamSynchronize(s));
    d.count = D.n_kv_heads;
    d.armed = true;
    return wait_done(kv, d);
}

// ---- decode ----------------------------------------------------------------------

int tq_hip_decode_async(tq_hip_kv *kv, int n_q, const int32_t *d_seq, const int32_t *d_len, int max_len,
                        const float *d_q, const float *d_cos, const float *d_sin, float *d_out,
                        void *stream) {
    if (!kv || n_q < 0) return TQ_HIP_EINVAL;
    if (n_q > 0 && !d_len) return TQ_HIP_EINVAL;
    if (!d_seq && n_q > kv->desc.max_seqs) return TQ_HIP_EINVAL;
    return decode_common(kv, n_q, d_seq, d_len, 0, 0, 1, 0, max_len, d_q, d_cos, d_sin, nullptr, nullptr,
                         d_out, pick(kv, stream), (!d_seq && n_q == 1) ? 0 : -1);
}

int tq_hip_decode_step_async(tq_hip_kv *kv, int n_q, const int32_t *d_seq, const int32_t *d_pos,
                             int max_pos, const float *d_q, const float *d_k, const float *d_v,
                             const float *d_cos, const float *d_sin, float *d_out, void *stream) {
    if (!kv || n_q < 0 || max_pos < 0) return TQ_HIP_EINVAL;
    if (n_q > 0 && (!d_pos || !d_k || !d_v)) return TQ_HIP_EINVAL;
    if (!d_seq && n_q > kv->desc.max_seqs) return TQ_HIP_EINVAL;
    return decode_common(kv, n_q, d_seq, d_pos, 1, 0, 1, 0, max_pos + 1, d_q, d_cos, d_sin, d_k, d_v, d_out,
                         pick(kv, stream), (!d_seq && n_q == 1) ? 0 : -1);
}

int tq_hip_decode_step_noalloc(tq_hip_kv *kv, int n_q, const int32_t *d_seq, const int32_t *d_pos, int max_pos,
                               const float *d_q, const float *d_k, const float *d_v, const float *d_cos,
                               const float *d_sin, float *d_out, void *stream) {
    if (!kv || n_q < 0 || max_pos < 0) return TQ_HIP_EINVAL;
    if (n_q > 0 && (!d_pos || !d_k || !d_v)) return TQ_HIP_EINVAL;
    if (!d_seq && n_q > kv->desc.max_seqs) return TQ_HIP_EINVAL;
    int dev = 0;
    TQ_TRY(hipGetDevice(&dev));
    const int rc = noalloc_setup(dev);
    if (rc != TQ_HIP_OK) return rc;
    unsigned char *base = g_noalloc[dev].ptr;
    const CallScratch sc{reinterpret_cast<float *>(base + kNoAllocCounterBytes),
                         TQ_HIP_NOALLOC_SCRATCH_BYTES - kNoAllocCounterBytes, reinterpret_cast<int *>(base),
                         kNoAllocCounterBytes / sizeof(int)};
    return decode_common(kv, n_q, d_seq, d_pos, 1, 0, 1, 0, max_pos + 1, d_q, d_cos, d_sin, d_k, d_v, d_out,
                         pick(kv, stream), (!d_seq && n_q == 1) ? 0 : -1, nullptr, nullptr, 0.0f, &sc);
}

int tq_hip_decode_step_norm_async(tq_hip_kv *kv, int n_q, const int32_t *d_seq, const int32_t *d_pos,
                                  int max_pos, const float *d_q, const float *d_k, const float *d_v,
                                  const float *d_q_norm, const float *d_k_norm, float rms_eps,
                                  const float *d_cos, const float *d_sin, float *d_out, void *stream) {
    if (!kv || n_q < 0 || max_pos < 0) return TQ_HIP_EINVAL;
    if (n_q > 0 && (!d_pos || !d_k || !d_v || !d_q_norm || !d_k_norm)) return TQ_HIP_EINVAL;
    if (!d_seq && n_q > kv->desc.max_seqs) return TQ_HIP_EINVAL;
    return decode_common(kv, n_q, d_seq, d_pos, 1, 0, 1, 0, max_pos + 1, d_q, d_cos, d_sin, d_k, d_v, d_out,
                         pick(kv, stream), (!d_seq && n_q == 1) ? 0 : -1, d_q_norm, d_k_norm, rms_eps);
}

int tq_hip_attend(tq_hip_kv *kv, int seq, int pos, const float *q, const float *cos_t, const float *sin_t,
                  float *out) {
    if (!seq_ok(kv, seq) || !q || !out || ((cos_t == nullptr) != (sin_t == nullptr))) return TQ_HIP_EINVAL;
    if (pos < 0 || pos >= capacity_of(kv, seq)) return TQ_HIP_EINVAL;
    const tq_hip_kv_desc &D = kv->desc;
    const size_t qb = (size_t)D.n_q_heads * D.head_dim * sizeof(float);
    const size_t tb = (size_t)(D.head_dim / 2) * sizeof(float);
    Stage st;
    const size_t oq = st.take(qb), oc = st.take(tb), os = st.take(tb);
    const size_t in_bytes = st.used, oo = st.take(qb);
    int rc = ensure_stage(kv, st.used);
    if (rc != TQ_HIP_OK) return rc;
    const hipStream_t s = kv->stream;
    unsigned char *S = nullptr;
    pack(kv, oq, q, qb);
    pack(kv, oc, cos_t, tb);
    pack(kv, os, sin_t, tb);
    rc = inputs_at(kv, in_bytes, true, &S);
    if (rc != TQ_HIP_OK) return rc;
    DoneFlags done;
    if (qb <= kDirectOut) done = next_done(kv);
    rc = decode_common(kv, 1, nullptr, nullptr, 0, seq, 0, pos, pos + 1, (const float *)(S + oq),
                       cos_t ? (const float *)(S + oc) : nullptr, cos_t ? (const float *)(S + os) : nullptr,
                       nullptr, nullptr, out_slot(kv, oo, qb), s, seq, nullptr, nullptr, 0.0f, nullptr, &done);
    if (rc != TQ_HIP_OK) return rc;
    return copy_out_sync(kv, out, oo, qb, &done);
}

// ---- prefill ---------------------------------------------------------------------

namespace {
// Whether a prefill of n tokens at these pointers takes the dense kernel.
bool prefill_takes_dense(const tq_hip_kv *kv, int pos0, int n, const float *d_q, const float *d_cos,
                         const float *d_sin, const float *d_out) {
    const tq_hip_kv_desc &D = kv->desc;
    const bool aligned16 = (((uintptr_t)d_q | (uintptr_t)d_cos | (uintptr_t)d_sin | (uintptr_t)d_out) & 15) == 0;
    return n > 1 && prefill_dense() && n >= kPrefillDenseMin && aligned16 &&
           tq_prefill_mfma_supported(D.head_dim, D.n_q_heads / D.n_kv_heads, pos0 + n);
}

// tq_hip_prefill_async; `done` (the synchronous entry point's completion
// flags) is armed when the decode form runs.  With q_norm / k_norm (16-byte
// aligned) the staging launch normalizes q and the new K rows itself; only
// the dense form with the fused append takes them (check prefill_fuses_norm).
int prefill_impl(tq_hip_kv *kv, int seq, int pos0, int n, const float *d_q, const float *d_k, const float *d_v,
                 const float *d_cos, const float *d_sin, float *d_out, hipStream_t s, DoneFlags *done,
                 const float *q_norm = nullptr, const float *k_norm = nullptr, float rms_eps = 0.0f,
                 unsigned char *out_xs = nullptr) {
    const tq_hip_kv_desc &D = kv->desc;
    // one token: store_kv + attend as the decode step, one launch
    // (model/attention_layer.c:221-236 with n == 1)
    if (n == 1 && !out_xs)
        return decode_common(kv, 1, nullptr, nullptr, 0, seq, 0, pos0, pos0 + 1, d_q, d_cos, d_sin, d_k, d_v,
                             d_out, s, seq, nullptr, nullptr, 0.0f, nullptr, done);
    // the dense kernel restages every key tile of [0, pos0+n): worth it from a
    // few dozen new tokens on; shorter batches attend in the decode form
    // the dense kernel moves q, cos/sin and out in 16-byte vectors; with 16-byte
    // aligned k and v its staging launch appends the new rows too
    const bool dense = prefill_takes_dense(kv, pos0, n, d_q, d_cos, d_sin, d_out);
    const bool fused = dense && (((uintptr_t)d_k | (uintptr_t)d_v) & 15) == 0;
    if (out_xs && !fused) return TQ_HIP_EINVAL;   // only the dense kernel quantizes its rows
    if (!fused)
        TQ_TRY(tq_launch_append(kv->view, n, nullptr, nullptr, seq, pos0, d_k, d_v, d_cos, d_sin,
                                kv->desc.head_dim, s));
    if (dense) {
        if (q_norm && !fused) return TQ_HIP_EINVAL;   // the caller checks prefill_fuses_norm first
        TqPrefillArgs t;
        t.k_new = fused ? d_k : nullptr;
        t.v_new = fused ? d_v : nullptr;
        t.q_norm = q_norm;
        t.k_norm = k_norm;
        t.rms_eps = rms_eps;
        t.out_xs = out_xs;
        t.view = kv->view;
        t.seq = seq;
        t.pos0 = pos0;
        t.n = n;
        t.q = d_q;
        t.cos_t = d_cos;
        t.sin_t = d_sin;
        t.out = d_out;
        t.n_q_heads = D.n_q_heads;
        t.n_kv_heads = D.n_kv_heads;
        t.head_dim = D.head_dim;
        t.scale = 1.0f / sqrtf((float)D.head_dim);
        int first = -1, pages = 0;
        seq_contig(kv, seq, &first, &pages);
        t.contig_first = pages > 0 ? first : -1;
        t.contig_pages = pages;
        int rc = ensure_img(kv, tq_prefill_image_bytes(D.head_dim, D.n_q_heads / D.n_kv_heads, D.n_kv_heads, pos0, n));
        if (rc != TQ_HIP_OK) return rc;
        size_t pbytes = 0, cn = 0;
        tq_prefill_scratch(D.head_dim, D.n_q_heads / D.n_kv_heads, D.n_kv_heads, pos0, n, &pbytes, &cn);
        rc = ensure_prefill_scratch(kv, std::max<size_t>(pbytes, 16), std::max<size_t>(cn, 1), s);
        if (rc != TQ_HIP_OK) return rc;
        t.img = kv->img;
        t.partials = kv->ppartials;
        t.counters = kv->pcounters;
        return herr(tq_launch_prefill(t, s));
    }
    if (q_norm) return TQ_HIP_EINVAL;
    return decode_common(kv, n, nullptr, nullptr, 0, seq, 0, pos0, pos0 + n, d_q, d_cos, d_sin, nullptr, nullptr,
                         d_out, s, seq, nullptr, nullptr, 0.0f, nullptr, done);
}

// Whether a prefill with these pointers takes the dense form with the append
// in its staging launch, which can normalize q and K too
// (TQ_HIP_PREFILL_FUSED_NORM=0 keeps the separate norm launches).
bool prefill_fuses_norm(const tq_hip_kv *kv, int pos0, int n, const float *d_q, const float *d_k, const float *d_v,
                        const float *d_cos, const float *d_sin, const float *d_out, const float *q_norm,
                        const float *k_norm) {
    const char *e = getenv("TQ_HIP_PREFILL_FUSED_NORM");
    const bool on = !(e && e[0] == '0');
    return on && prefill_takes_dense(kv, pos0, n, d_q, d_cos, d_sin, d_out) &&
           (((uintptr_t)d_k | (uintptr_t)d_v | (uintptr_t)q_norm | (uintptr_t)k_norm) & 15) == 0;
}
}  // namespace

int tq_hip_prefill_async(tq_hip_kv *kv, int seq, int pos0, int n, const float *d_q, const float *d_k,
                         const float *d_v, const float *d_cos, const float *d_sin, float *d_out,
                         void *stream) {
    if (!seq_ok(kv, seq) || !d_q || !d_k || !d_v || !d_out || ((d_cos == nullptr) != (d_sin == nullptr)))
        return TQ_HIP_EINVAL;
    // model/attention_layer.c:203-204
    if (n <= 0 || pos0 < 0 || pos0 + n > capacity_of(kv, seq)) return TQ_HIP_EINVAL;
    return prefill_impl(kv, seq, pos0, n, d_q, d_k, d_v, d_cos, d_sin, d_out, pick(kv, stream), nullptr);
}

int tq_hip_prefill(tq_hip_kv *kv, int seq, int pos0, int n, const float *q, const float *k, const float *v,
                   const float *cos_t, const float *sin_t, float *out) {
    if (!seq_ok(kv, seq) || !q || !k || !v || !out || ((cos_t == nullptr) != (sin_t == nullptr)))
        return TQ_HIP_EINVAL;
    if (n <= 0 || pos0 < 0 || pos0 + n > capacity_of(kv, seq)) return TQ_HIP_EINVAL;
    const tq_hip_kv_desc &D = kv->desc;
    const size_t qb = (size_t)n * D.n_q_heads * D.head_dim * sizeof(float);
    const size_t kvb = (size_t)n * D.n_kv_heads * D.head_dim * sizeof(float);
    const size_t tb = (size_t)n * (D.head_dim / 2) * sizeof(float);
    Stage st;
    const size_t oq = st.take(qb), ok_ = st.take(kvb), ov = st.take(kvb), oc = st.take(tb), os = st.take(tb);
    const size_t in_bytes = st.used, oo = st.take(qb);
    int rc = ensure_stage(kv, st.used);
    if (rc != TQ_HIP_OK) return rc;
    const hipStream_t s = kv->stream;
    pack(kv, oq, q, qb);
    pack(kv, ok_, k, kvb);
    pack(kv, ov, v, kvb);
    pack(kv, oc, cos_t, tb);
    pack(kv, os, sin_t, tb);
    // the decode form may read its inputs in host memory; the dense kernel
    // streams them and takes the device copy (the staging offsets are 256-byte
    // aligned in both, so the choice of form does not depend on it)
    float *o = out_slot(kv, oo, qb);
    const bool dense = prefill_takes_dense(kv, pos0, n, reinterpret_cast<const float *>(kv->stage + oq),
                                           reinterpret_cast<const float *>(kv->stage + oc),
                                           reinterpret_cast<const float *>(kv->stage + os), o);
    unsigned char *S = nullptr;
    rc = inputs_at(kv, in_bytes, !dense, &S);
    if (rc != TQ_HIP_OK) return rc;
    DoneFlags done;
    if (!dense && qb <= kDirectOut) done = next_done(kv);
    rc = prefill_impl(kv, seq, pos0, n, (const float *)(S + oq), (const float *)(S + ok_), (const float *)(S + ov),
                      cos_t ? (const float *)(S + oc) : nullptr, cos_t ? (const float *)(S + os) : nullptr, o, s,
                      &done);
    if (rc != TQ_HIP_OK) return rc;
    return copy_out_sync(kv, out, oo, qb, &done);
}


// ---- the whole attention layer -------------------------------------------

static size_t layer_ws(const tq_hip_kv_desc &D, int hidden, int n_q, size_t *off_q, size_t *off_k,
                       size_t *off_v, size_t *off_attn, size_t *off_xq, size_t *off_part = nullptr,
                       size_t *part_floats = nullptr) {
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const size_t qd = (size_t)D.n_q_heads * D.head_dim, kd = (size_t)D.n_kv_heads * D.head_dim;
    const size_t widest = (size_t)(hidden > (int)qd ? hidden : (int)qd);
    size_t o = 0;
    *off_q = o;
    o += al((size_t)n_q * qd * 4);
    *off_k = o;
    o += al((size_t)n_q * kd * 4);
    *off_v = o;
    o += al((size_t)n_q * kd * 4);
    *off_attn = o;
    o += al((size_t)n_q * qd * 4);
    *off_xq = o;
    o += al((size_t)n_q * widest / QK * sizeof(block_q8));
    // split-K partials of the q/k/v and the output matmuls (one at a time)
    const size_t pq = tq_gemm_partial_floats((int)(qd + 2 * kd), hidden, n_q);
    const size_t po = tq_gemm_partial_floats(hidden, (int)qd, n_q);
    const size_t pf = pq > po ? pq : po;
    if (off_part) *off_part = o;
    if (part_floats) *part_floats = pf;
    o += al(pf * 4);
    return o;
}

static bool layer_shape_ok(const tq_hip_kv *kv, const tq_hip_attn_weights *w, int n_q) {
    return kv && w && n_q > 0 && w->hidden > 0 && w->hidden % QK == 0 &&
           (kv->desc.n_q_heads * kv->desc.head_dim) % QK == 0 &&
           (w->format == TQ_HIP_FORMAT_Q8 || w->format == TQ_HIP_FORMAT_Q4);
}

size_t tq_hip_attention_layer_ws_bytes(const tq_hip_kv *kv, const tq_hip_attn_weights *w, int n_q) {
    if (!layer_shape_ok(kv, w, n_q)) return 0;
    size_t oq, ok, ov, oa, ox;
    return layer_ws(kv->desc, w->hidden, n_q, &oq, &ok, &ov, &oa, &ox);
}

int tq_hip_attention_layer_async(tq_hip_kv *kv, const tq_hip_attn_weights *w, int n_q,
                                 const int32_t *d_seq, const int32_t *d_pos, int max_pos,
                                 const float *d_xn, const float *d_cos, const float *d_sin,
                                 float *d_out, void *d_ws, size_t ws_bytes, void *stream) {
    if (!layer_shape_ok(kv, w, n_q) || !d_pos || !d_xn || !d_out || !d_ws || ((uintptr_t)d_ws & 15) ||
        !w->wq || !w->wk || !w->wv || !w->wo || !w->q_norm || !w->k_norm)
        return TQ_HIP_EINVAL;
    const tq_hip_kv_desc &D = kv->desc;
    size_t oq, ok, ov, oa, ox, op, pf;
    if (ws_bytes < layer_ws(D, w->hidden, n_q, &oq, &ok, &ov, &oa, &ox, &op, &pf)) return TQ_HIP_EINVAL;
    unsigned char *ws = (unsigned char *)d_ws;
    float *q = (float *)(ws + oq), *k = (float *)(ws + ok), *v = (float *)(ws + ov);
    float *attn = (float *)(ws + oa);
    block_q8 *xq = (block_q8 *)(ws + ox);
    float *part = (float *)(ws + op);
    const int qd = D.n_q_heads * D.head_dim, kd = D.n_kv_heads * D.head_dim;
    void *s = (void *)pick(kv, stream);
    const bool q4 = w->format == TQ_HIP_FORMAT_Q4;
    int rc = tq_project_qkv_fmt(q4, w->wq, w->wk, w->wv, qd, kd, w->hidden, d_xn, n_q, xq, q, k, v, s, part, pf);
    if (rc != TQ_HIP_OK) return rc;
    rc = tq_hip_decode_step_norm_async(kv, n_q, d_seq, d_pos, max_pos, q, k, v, w->q_norm, w->k_norm,
                                       w->rms_eps, d_cos, d_sin, attn, s);
    if (rc != TQ_HIP_OK) return rc;
    return tq_project_output_fmt(q4, w->wo, w->hidden, qd, attn, n_q, xq, d_out, s, part, pf);
}

int tq_hip_attention_layer_batch_async(tq_hip_kv *kv, const tq_hip_attn_weights *w, int seq, int pos0,
                                       int n, const float *d_xn, const float *d_cos, const float *d_sin,
                                       float *d_out, void *d_ws, size_t ws_bytes, void *stream) {
    if (!layer_shape_ok(kv, w, n) || !seq_ok(kv, seq) || !d_xn || !d_out || !d_ws || ((uintptr_t)d_ws & 15) ||
        !w->wq || !w->wk || !w->wv || !w->wo || !w->q_norm || !w->k_norm ||
        ((d_cos == nullptr) != (d_sin == nullptr)))
        return TQ_HIP_EINVAL;
    // model/attention_layer.c:203-204
    if (pos0 < 0 || pos0 + n > capacity_of(kv, seq)) return TQ_HIP_EINVAL;
    const tq_hip_kv_desc &D = kv->desc;
    size_t oq, ok, ov, oa, ox, op, pf;
    if (ws_bytes < layer_ws(D, w->hidden, n, &oq, &ok, &ov, &oa, &ox, &op, &pf)) return TQ_HIP_EINVAL;
    unsigned char *ws = (unsigned char *)d_ws;
    float *q = (float *)(ws + oq), *k = (float *)(ws + ok), *v = (float *)(ws + ov);
    float *attn = (float *)(ws + oa);
    block_q8 *xq = (block_q8 *)(ws + ox);
    float *part = (float *)(ws + op);
    const int qd = D.n_q_heads * D.head_dim, kd = D.n_kv_heads * D.head_dim;
    const hipStream_t hs = pick(kv, stream);
    void *s = (void *)hs;
    // :213-218 quantize every row, then the batched q/k/v projections
    const bool q4 = w->format == TQ_HIP_FORMAT_Q4;
    int rc = tq_project_qkv_fmt(q4, w->wq, w->wk, w->wv, qd, kd, w->hidden, d_xn, n, xq, q, k, v, s, part, pf);
    if (rc != TQ_HIP_OK) return rc;
    // :227-228 norm_heads on every token's q and k rows: in the prefill's
    // staging launch where it takes them, else two row launches
    if (prefill_fuses_norm(kv, pos0, n, q, k, v, d_cos, d_sin, attn, w->q_norm, w->k_norm)) {
        // :230-235 RoPE, store_kv and causal attention for the n tokens; when
        // the output projection is a GEMM over the split layout, the prefill
        // quantizes its rows straight into that layout (:238's quantization,
        // TQ_HIP_PREFILL_QUANT_OUT=0 keeps the fp32 rows and a separate launch)
        const char *e = getenv("TQ_HIP_PREFILL_QUANT_OUT");
        const bool qout = !(e && e[0] == '0') &&
                          tq_project_output_takes_xs(q4, w->wo, w->hidden, qd, n, xq, part, pf);
        rc = prefill_impl(kv, seq, pos0, n, q, k, v, d_cos, d_sin, attn, hs, nullptr, w->q_norm, w->k_norm,
                          w->rms_eps, qout ? (unsigned char *)xq : nullptr);
        if (rc != TQ_HIP_OK) return rc;
        if (qout) return tq_project_output_xs(q4, w->wo, w->hidden, qd, xq, n, d_out, s, part, pf);
    } else {
        TQ_TRY(tq_launch_rmsnorm_rows(q, w->q_norm, q, n * D.n_q_heads, D.head_dim, w->rms_eps, hs));
        TQ_TRY(tq_launch_rmsnorm_rows(k, w->k_norm, k, n * D.n_kv_heads, D.head_dim, w->rms_eps, hs));
        rc = tq_hip_prefill_async(kv, seq, pos0, n, q, k, v, d_cos, d_sin, attn, s);
    }
    if (rc != TQ_HIP_OK) return rc;
    // :238-241 quantize the attention rows, then the batched output projection
    return tq_project_output_fmt(q4, w->wo, w->hidden, qd, attn, n, xq, d_out, s, part, pf);
}

}  // extern "C"
