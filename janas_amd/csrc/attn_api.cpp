/*
 * attn_api.cpp - the C ABI of include/janas_attn.h over the HIP kernels.
 *
 * The instance mirrors the reference's struct janas_attn
 * (src/llm/attention.c:37-58): geometry, scale, window, ring, sixteen-bit
 * cache, the next call's last positions; what the reference keeps in host
 * memory (partials) lives on the device, with the stream the calls run on.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <sys/stat.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <vector>

#include <hip/hip_runtime.h>

#include "../../include/janas_attn.h"
#include "attn_kernels.h"

using namespace janas;

namespace {

struct ProfEv {
    int kind;
    hipEvent_t a, b;
};

/* host bytes [host, host + bytes) and their device copy (janas_attn_import) */
struct HostCopy {
    const char *host;
    size_t bytes;
    char *dev;
};

}  // namespace

struct janas_attn {
    uint32_t n_head, n_kv, hd, n_ctx, group;
    int scores;           /* JANAS_ATTN_FLOAT or _INT16, as resolved */
    int scores_auto;
    /* AUTO over int8 caches: INT16 from position from16[n > 1] on,
       measured on the device at the first call (calibrate) */
    uint32_t from16[2];
    int calibrated;
    float scale;
    uint32_t window;
    int kv16, ring;
    const uint32_t *last; /* host, the next janas_attn_run only */
    int dev;
    uint32_t cus;         /* compute units of the device */
    hipStream_t stream;
    /* partials: part_rows rows of (m, l) and of hd values */
    float *part_ml, *part_acc;
    uint64_t part_rows;
    /* the stream that last used the partials: a call on another stream
       waits for its work first (part_ev), and the partials are freed only
       once it is done */
    hipStream_t part_stream;
    hipEvent_t part_ev;
    /* the exact prefill kernel's copies of an int8 / int16 cache's keys
       and values as f16 planes (dq_bytes each), ordered across streams as
       the partials */
    void *dq_k, *dq_v;
    size_t dq_bytes;
    /* staging of host pointers for janas_attn_run, and the bytes each
       staging buffer holds */
    float *st_q, *st_out;
    void *st_k, *st_v;
    float *st_ks, *st_vs;
    uint32_t *st_last;
    size_t st_k_bytes, st_v_bytes, st_ks_bytes, st_vs_bytes;
    /* the first device failure since create (or the last clear): sticky;
       abort_on_error: janas_attn_run aborts on one (the default) */
    int status;
    int abort_on_error;
    /* timing */
    int prof;
    std::vector<ProfEv> *ev_used, *ev_free;
    /* imported host ranges (janas_attn_import) */
    std::vector<HostCopy> *copies;
    /* pinned host memory for what a janas_attn_run with host pointers
       sends and receives besides a staged cache: q, the rows of imported
       caches, out */
    char *pin;
    size_t pin_bytes;
};

namespace {

int hip_err(hipError_t e, const char *what)
{
    if (e == hipSuccess)
        return JANAS_ATTN_OK;
    fprintf(stderr, "janas_attn: %s: %s\n", what, hipGetErrorString(e));
    return JANAS_ATTN_EDEVICE;
}

bool is_device_ptr(const void *p)
{
    if (!p)
        return false;
    hipPointerAttribute_t at;
    hipError_t e = hipPointerGetAttributes(&at, p);
    if (e != hipSuccess) {
        (void)hipGetLastError(); /* an unregistered host pointer */
        return false;
    }
    return at.type == hipMemoryTypeDevice || at.type == hipMemoryTypeManaged;
}

/* the imported range holding host bytes [p, p + bytes), or null */
const HostCopy *find_copy(const janas_attn *a, const void *p, size_t bytes)
{
    const char *q = (const char *)p;
    for (const HostCopy &c : *a->copies)
        if (q >= c.host && bytes <= c.bytes && (size_t)(q - c.host) <= c.bytes - bytes)
            return &c;
    return nullptr;
}

/* A call over an imported cache: the rows of positions [pos0, end) (p mod
   cap in a ring), each KV head, from the host to the device copy - the rows
   the call's tokens were just written to. esz: bytes a row. */
int refresh_rows(janas_attn *a, char *dev, const void *host, size_t esz,
                 uint32_t pos0, uint32_t end)
{
    const size_t cap = a->n_ctx, pitch = cap * esz;
    size_t lo = a->ring ? pos0 % cap : pos0, n = end - pos0;
    if (n > cap)
        n = cap;
    while (n) {
        const size_t run = std::min(n, cap - lo);
        int rc = hip_err(hipMemcpy2DAsync(dev + lo * esz, pitch, (const char *)host + lo * esz,
                                          pitch, run * esz, a->n_kv, hipMemcpyHostToDevice,
                                          a->stream),
                         "copy the call's rows");
        if (rc)
            return rc;
        n -= run;
        lo = 0;
    }
    return JANAS_ATTN_OK;
}

uint32_t elem_bytes(int kv)
{
    return kv == kI8 ? 1 : kv == kF32 ? 4 : 2;
}

uint32_t first_chunk(uint32_t window, uint32_t pos0)
{
    return window && pos0 + 1 > window ? (pos0 + 1 - window) / kChunk : 0;
}

/* Fill the kernel view of one sequence and check it against the cache. */
int describe(const janas_attn *a, int kv, const janas_attn_seq &s, SeqDesc &d)
{
    if (!s.k || !s.v || !s.q || !s.out || s.n == 0 || s.cap == 0)
        return JANAS_ATTN_EINVAL;
    if ((kv == kI8 || kv == kI16) && (!s.ks || !s.vs))
        return JANAS_ATTN_EINVAL;
    /* the kernels count a sequence's query rows (n x heads) in 32 bits */
    if ((uint64_t)s.n * a->n_head > 0x7FFFFFFFu)
        return JANAS_ATTN_ERANGE;
    memset(&d, 0, sizeof d);
    d.k = s.k;
    d.v = s.v;
    d.ks = s.ks;
    d.vs = s.vs;
    d.q = s.q;
    d.out = s.out;
    d.gate = s.gate;
    d.last = s.last;
    d.cap = s.cap;
    d.n = s.n;
    d.pos0 = s.pos0;
    if (s.last && s.last_max < s.pos0 + s.n - 1)
        return JANAS_ATTN_EINVAL;
    uint64_t end = s.last ? (uint64_t)s.last_max + 1 : (uint64_t)s.pos0 + s.n;
    if (end > 0xFFFFFF00u)
        return JANAS_ATTN_ERANGE;
    d.end = (uint32_t)end;
    d.c0 = first_chunk(a->window, s.pos0);
    uint32_t n_chunks = (d.end + kChunk - 1) / kChunk;
    d.span = n_chunks - d.c0;
    if (a->ring) {
        /* attention.c:1281-1286: the call must fit in the ring */
        if (s.cap % kChunk || d.span * kChunk > s.cap)
            return JANAS_ATTN_ERANGE;
    } else if (d.end > s.cap) {
        return JANAS_ATTN_ERANGE;
    }
    const uint32_t tr = split_tile_rows(a->hd);
    d.rtiles = (s.n * a->group + tr - 1) / tr;
    if (s.out_q8k && ((uint64_t)a->n_head * a->hd) % JANAS_ATTN_QK)
        return JANAS_ATTN_EINVAL;
    d.q8k = s.out_q8k;
    return JANAS_ATTN_OK;
}

/* The outputs also as Q8_K blocks where a sequence asks for them
   (att_out_tok, model_attn.c:159-170: the gate is already in the output):
   the prefill path's pass over its outputs (the split path's merge
   quantizes its own). */
int put_q8k(const janas_attn *a, const janas_attn_seq *seqs, uint32_t n_seqs,
            hipStream_t stream)
{
    for (uint32_t i = 0; i < n_seqs; i++) {
        if (!seqs[i].out_q8k)
            continue;
        Q8kArgs q;
        q.x = seqs[i].out;
        q.y = (uint8_t *)seqs[i].out_q8k;
        uint64_t blocks = (uint64_t)seqs[i].n * a->n_head * a->hd / JANAS_ATTN_QK;
        if (blocks > 0x7FFFFFFFu)
            return JANAS_ATTN_ERANGE;
        q.blocks = (uint32_t)blocks;
        hipError_t e = launch_q8k(q, stream);
        if (e != hipSuccess)
            return hip_err(e, "q8k launch");
    }
    return JANAS_ATTN_OK;
}

/* A device failure is remembered (janas_attn_status) as well as returned. */
int note(janas_attn *a, int rc)
{
    if (rc && !a->status && rc != JANAS_ATTN_EINVAL && rc != JANAS_ATTN_ERANGE &&
        rc != JANAS_ATTN_ENOTSUP)
        a->status = rc;
    return rc;
}

/* The partials are about to be used on `stream`: if another stream used
   them last, this one first waits for everything queued there so far. */
int part_sync(janas_attn *a, hipStream_t stream)
{
    if (a->part_stream != stream) {
        if (a->part_stream) {
            hipError_t e = hipEventRecord(a->part_ev, a->part_stream);
            if (e == hipSuccess)
                e = hipStreamWaitEvent(stream, a->part_ev, 0);
            if (e != hipSuccess)
                return hip_err(e, "order the partials' streams");
        }
        a->part_stream = stream;
    }
    return JANAS_ATTN_OK;
}

int ensure_part(janas_attn *a, uint64_t rows, hipStream_t stream)
{
    if (rows <= a->part_rows)
        return JANAS_ATTN_OK;
    /* the stream that used them last, and this one, may still read the
       old ones */
    if (a->part_ml || a->part_acc) {
        hipError_t e = hipStreamSynchronize(stream);
        if (e == hipSuccess && a->part_stream && a->part_stream != stream)
            e = hipStreamSynchronize(a->part_stream);
        if (e != hipSuccess)
            return hip_err(e, "synchronize");
        (void)hipFree(a->part_ml);
        (void)hipFree(a->part_acc);
        a->part_ml = a->part_acc = nullptr;
        a->part_rows = 0;
    }
    if (hipMalloc(&a->part_ml, rows * 2 * sizeof(float)) != hipSuccess ||
        hipMalloc(&a->part_acc, rows * a->hd * sizeof(float)) != hipSuccess) {
        (void)hipGetLastError();
        (void)hipFree(a->part_ml);
        (void)hipFree(a->part_acc);
        a->part_ml = a->part_acc = nullptr;
        return JANAS_ATTN_ENOMEM;
    }
    a->part_rows = rows;
    return JANAS_ATTN_OK;
}

/* Where a call's partials live: the instance's (grown as needed, ordered
   across streams), or the device's fixed array of the allocation-free
   entry point (a call that needs more rows is refused). */
struct Parts {
    float *ml, *acc;
    bool fixed;
};

int get_parts(janas_attn *a, uint64_t rows, hipStream_t stream, bool fixed, Parts &p,
              uint64_t reserve = 0)
{
    if (fixed) {
        /* past the first `reserve` bytes of the array (a prompt's exact
           copy, 256-byte aligned) */
        char *base = (char *)scratch_ptr(a->dev);
        if (!base)
            return JANAS_ATTN_EDEVICE;
        /* ml: rows x 2 floats, then acc (256-byte aligned): rows x hd */
        const uint64_t ml_bytes = (rows * 2 * sizeof(float) + 255) / 256 * 256;
        if (reserve + ml_bytes + rows * a->hd * sizeof(float) > JANAS_ATTN_NOALLOC_BYTES)
            return JANAS_ATTN_ERANGE;
        p.ml = (float *)(base + reserve);
        p.acc = (float *)(base + reserve + ml_bytes);
        p.fixed = true;
        return JANAS_ATTN_OK;
    }
    int rc = ensure_part(a, rows, stream);
    if (!rc)
        rc = part_sync(a, stream);
    p.ml = a->part_ml;
    p.acc = a->part_acc;
    p.fixed = false;
    return rc;
}

ProfEv *prof_begin(janas_attn *a, int kind, hipStream_t stream)
{
    if (!a->prof)
        return nullptr;
    ProfEv ev;
    if (!a->ev_free->empty()) {
        ev = a->ev_free->back();
        a->ev_free->pop_back();
    } else if (hipEventCreate(&ev.a) != hipSuccess ||
               hipEventCreate(&ev.b) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    ev.kind = kind;
    a->ev_used->push_back(ev);
    (void)hipEventRecord(a->ev_used->back().a, stream);
    return &a->ev_used->back();
}

void prof_end(ProfEv *ev, hipStream_t stream)
{
    if (ev)
        (void)hipEventRecord(ev->b, stream);
}

/* JANAS_ATTN_SKIPSTAT=1 (attention.c:841-869, :1320-1325): how many
   chunks a row could have skipped, had it known in advance which ones
   weigh nothing - their largest score more than 8, 16 or 32 below the
   row's - printed when the program ends, over all rows and over those past
   16384 positions. Read at the first janas_attn_create of the process;
   counted by the merge of the split path (decode, verify, blocks), on the
   device, into counters each device holds from that create on. The
   prefill kernels keep no chunk partials and are not counted. */
constexpr int kSkipDevs = 64;
int g_skip = -1;
unsigned long long *g_skip_dev[kSkipDevs];

void skip_report()
{
    static const char *what[2] = {"all rows", "rows past 16384"};
    unsigned long long t[8] = {0};
    for (int d = 0; d < kSkipDevs; d++) {
        unsigned long long h[8];
        if (!g_skip_dev[d] || hipSetDevice(d) != hipSuccess ||
            hipMemcpy(h, g_skip_dev[d], sizeof h, hipMemcpyDeviceToHost) != hipSuccess)
            continue;
        for (int i = 0; i < 8; i++)
            t[i] += h[i];
    }
    for (int w = 0; w < 2; w++) {
        const unsigned long long n = t[w];
        if (!n)
            continue;
        fprintf(stderr,
                "attention skip ceiling, %s: %llu chunks; below max-8 "
                "%.1f%%, max-16 %.1f%%, max-32 %.1f%%\n",
                what[w], n, 100.0 * t[2 + 3 * w] / n, 100.0 * t[3 + 3 * w] / n,
                100.0 * t[4 + 3 * w] / n);
    }
}

/* the counters of device dev, allocated at a create on it (null: off, or
   the allocation failed, which leaves the statistic off there) */
void skip_init(int dev)
{
    if (g_skip < 0) {
        const char *e = getenv("JANAS_ATTN_SKIPSTAT");
        g_skip = e && atoi(e) > 0;
        if (g_skip)
            atexit(skip_report);
    }
    if (!g_skip || dev < 0 || dev >= kSkipDevs || g_skip_dev[dev])
        return;
    unsigned long long *p = nullptr;
    if (hipMalloc(&p, 8 * sizeof *p) != hipSuccess || hipMemset(p, 0, 8 * sizeof *p) != hipSuccess) {
        (void)hipGetLastError();
        (void)hipFree(p);
        return;
    }
    g_skip_dev[dev] = p;
}

int fill_args(const janas_attn *a, int kv, SplitArgs &args, int gate_mode, const Parts &p)
{
    args.skip = g_skip > 0 && a->dev >= 0 && a->dev < kSkipDevs ? g_skip_dev[a->dev] : nullptr;
    /* the INT16 way exists over int8 caches (attention.c:692, :1061-1066) */
    args.int16 = kv == kI8 && a->scores == JANAS_ATTN_INT16;
    args.part_ml = p.ml;
    args.part_acc = p.acc;
    args.n_head = a->n_head;
    args.n_kv = a->n_kv;
    args.group = a->group;
    args.hd = a->hd;
    args.window = a->window;
    args.scale = a->scale;
    args.ring = a->ring;
    args.gate_mode = gate_mode;
    return JANAS_ATTN_OK;
}

int run_split(janas_attn *a, int kv, int gate_mode, const janas_attn_seq *seqs,
              uint32_t n_seqs, hipStream_t stream, int kernels = 3, bool fixed = false)
{
    if (!split_supported(kv, a->hd))
        return JANAS_ATTN_ENOTSUP;
    for (uint32_t s0 = 0; s0 < n_seqs; s0 += kMaxSeqs) {
        uint32_t m = std::min(kMaxSeqs, n_seqs - s0);
        SplitArgs args;
        memset(&args, 0, sizeof args);
        uint64_t rows = 0, pairs = 0;
        bool q8k = false;
        for (uint32_t i = 0; i < m; i++) {
            pairs += (uint64_t)seqs[s0 + i].n * a->n_head;
            q8k |= seqs[s0 + i].out_q8k != nullptr;
        }
        /* a sequence that asks for Q8_K blocks: the merge takes a block a
           workgroup and quantizes it (the same output bits) */
        args.merge_cols = q8k ? kMergeQ8k : merge_cols(pairs, a->hd);
        /* row tiles a workgroup, from the launch's largest sequence */
        const uint32_t tr = split_tile_rows(a->hd);
        uint64_t tiles = 1;
        for (uint32_t i = 0; i < m; i++)
            tiles = std::max<uint64_t>(tiles, ((uint64_t)seqs[s0 + i].n * a->group + tr - 1) / tr);
        args.mt = split_mt(kv, a->hd, (uint32_t)std::min<uint64_t>(tiles, kSplitMaxMt));
        args.once = 1;
        uint32_t wg = 0, mg = 0;
        /* merge workgroups a (token, head), or a token's blocks */
        const uint32_t nd = (a->hd + args.merge_cols - 1) / args.merge_cols;
        const uint32_t nb = (uint32_t)((uint64_t)a->n_head * a->hd / JANAS_ATTN_QK);
        for (uint32_t i = 0; i < m; i++) {
            SeqDesc &d = args.seq[i];
            int rc = describe(a, kv, seqs[s0 + i], d);
            if (rc)
                return rc;
            d.wg0 = args.wg0s[i] = wg;
            d.mg0 = args.mg0s[i] = mg;
            d.part0 = rows;
            d.rtiles = (d.rtiles + args.mt - 1) / args.mt;
            args.once &= d.rtiles == 1;
            uint64_t nwg = (uint64_t)a->n_kv * d.span * d.rtiles;
            uint64_t nmg = q8k ? (uint64_t)d.n * nb : (uint64_t)d.n * a->n_head * nd;
            if (wg + nwg > 0x7FFFFFFFu || mg + nmg > 0x7FFFFFFFu)
                return JANAS_ATTN_ERANGE;
            wg += (uint32_t)nwg;
            mg += (uint32_t)nmg;
            rows += (uint64_t)a->n_kv * d.span * d.n * a->group;
        }
        Parts pt;
        int rc = get_parts(a, rows, stream, fixed, pt);
        if (rc)
            return rc;
        args.n_seqs = m;
        args.n_wg = wg;
        fill_args(a, kv, args, gate_mode, pt);
        if (kernels & 1) {
            ProfEv *ev = fixed ? nullptr : prof_begin(a, 0, stream);
            hipError_t e = launch_split(kv, args, stream);
            prof_end(ev, stream);
            if (e != hipSuccess)
                return hip_err(e, "split launch");
        }
        if (kernels & 2) {
            ProfEv *ev = fixed ? nullptr : prof_begin(a, 1, stream);
            hipError_t e = launch_merge(args, mg, stream);
            prof_end(ev, stream);
            if (e != hipSuccess)
                return hip_err(e, "merge launch");
        }
    }
    return JANAS_ATTN_OK;
}

/*
 * AUTO's way, measured (attn_calibrate, attention.c:1183-1262): over a
 * made-up int8 cache of this instance's geometry (as far as 65536 + 64
 * positions, a ring its whole capacity), one token at positions 1024,
 * 2048, ... up to 65536 and a 64-token block up to 16384 are timed both
 * ways on the device (the faster of three calls each, HIP events on the
 * instance's stream); INT16 is taken from the first position from which it
 * wins at every longer one. As the reference keeps its measurements in
 * attn.txt under its cache directory (attention.c:1118-1164, tuner.c:
 * 343-365), these are kept for the process and in attn_gpu.txt there
 * ($XDG_CACHE_HOME/janas, else ~/.cache/janas): one line a measurement,
 * "key from16[0] from16[1]", the key naming the device (its name,
 * architecture and compute units) and the geometry, so every later process
 * on the same kind of device takes it without measuring. On gfx950 INT16
 * costs 5-8 % more than FLOAT at every length, so AUTO measures to FLOAT.
 */
struct Calib {
    int dev, ring;
    uint32_t n_head, n_kv, hd, window, n_ctx;
    uint32_t from16[2];
};
std::mutex g_calib_mu;
std::vector<Calib> *g_calib;

bool calib_same(const Calib &c, const janas_attn *a)
{
    return c.dev == a->dev && c.ring == a->ring && c.n_head == a->n_head && c.n_kv == a->n_kv &&
           c.hd == a->hd && c.window == a->window && c.n_ctx == a->n_ctx;
}

/* the measurement's key: device, then geometry (no blanks) */
std::string calib_key(const janas_attn *a)
{
    hipDeviceProp_t pr;
    std::string dev = "gpu";
    if (hipGetDeviceProperties(&pr, a->dev) == hipSuccess)
        dev = std::string(pr.name) + "|" + pr.gcnArchName + "|" +
              std::to_string(pr.multiProcessorCount);
    else
        (void)hipGetLastError();
    for (char &c : dev)
        if (c == ' ' || c == '\t' || c == '\n')
            c = '_';
    char geo[160];
    snprintf(geo, sizeof geo, "|%d|%u/%u/%u|%u|%u", a->ring, a->n_head, a->n_kv, a->hd,
             a->window, a->n_ctx);
    return dev + geo;
}

/* the cache directory's file (tuner.c:343-365's directory), made if
   `create`; empty when there is no home */
std::string calib_path(bool create)
{
    const char *xdg = getenv("XDG_CACHE_HOME"), *home = getenv("HOME");
    std::string dir = xdg && *xdg ? std::string(xdg) + "/janas"
                    : home        ? std::string(home) + "/.cache/janas"
                                  : std::string();
    if (dir.empty())
        return dir;
    if (create)
        for (size_t i = 1; i <= dir.size(); i++)
            if (i == dir.size() || dir[i] == '/')
                (void)mkdir(dir.substr(0, i).c_str(), 0755);
    return dir + "/attn_gpu.txt";
}

/* the last line for `key` (later lines win, as appended), or false */
bool calib_load(const std::string &key, uint32_t from16[2])
{
    const std::string path = calib_path(false);
    FILE *f = path.empty() ? nullptr : fopen(path.c_str(), "r");
    if (!f)
        return false;
    bool found = false;
    char line[1024], k[800];
    while (fgets(line, sizeof line, f)) {
        unsigned x, y;
        if (sscanf(line, "%799s %u %u", k, &x, &y) == 3 && key == k) {
            from16[0] = x;
            from16[1] = y;
            found = true;
        }
    }
    fclose(f);
    return found;
}

void calib_save(const std::string &key, const uint32_t from16[2])
{
    const std::string path = calib_path(true);
    FILE *f = path.empty() ? nullptr : fopen(path.c_str(), "a");
    if (!f)
        return;
    fprintf(f, "%s %u %u\n", key.c_str(), from16[0], from16[1]);
    fclose(f);
}

/* milliseconds of the faster of three calls of this way, or -1 */
float time_way(janas_attn *a, int way, const janas_attn_seq &s, hipEvent_t e0, hipEvent_t e1)
{
    float best = 1e30f;
    a->scores = way;
    for (int r = 0; r < 3; r++) {
        if (hipEventRecord(e0, a->stream) != hipSuccess)
            return -1.0f;
        const int rc = run_split(a, kI8, kGateNone, &s, 1, a->stream);
        if (rc || hipEventRecord(e1, a->stream) != hipSuccess ||
            hipEventSynchronize(e1) != hipSuccess)
            return -1.0f;
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, e0, e1) != hipSuccess)
            return -1.0f;
        best = std::min(best, ms);
    }
    return best;
}

void calibrate(janas_attn *a)
{
    a->calibrated = 1;
    const uint64_t rows0 = a->part_rows;
    a->from16[0] = a->from16[1] = UINT32_MAX;
    const std::string key = calib_key(a);
    {
        std::lock_guard<std::mutex> lk(g_calib_mu);
        if (g_calib)
            for (const Calib &c : *g_calib)
                if (calib_same(c, a)) {
                    a->from16[0] = c.from16[0];
                    a->from16[1] = c.from16[1];
                    return;
                }
        if (calib_load(key, a->from16)) {
            if (!g_calib)
                g_calib = new std::vector<Calib>();
            g_calib->push_back(Calib{a->dev, a->ring, a->n_head, a->n_kv, a->hd, a->window,
                                     a->n_ctx, {a->from16[0], a->from16[1]}});
            return;
        }
    }
    const uint32_t nb = JANAS_ATTN_MAX_BLOCK < 64 ? JANAS_ATTN_MAX_BLOCK : 64;
    const uint32_t top = !a->ring && a->n_ctx > 65536 + nb ? 65536 + nb : a->n_ctx;
    const size_t cells = (size_t)a->n_kv * top;
    const size_t qn = (size_t)nb * a->n_head * a->hd;
    void *k = nullptr, *v = nullptr, *ks = nullptr, *vs = nullptr, *q = nullptr, *out = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    const int keep = a->scores;
    /* the measurement's own launches are not the caller's to count */
    const int prof = a->prof;
    a->prof = 0;
    bool ok = hipMalloc(&k, cells * a->hd) == hipSuccess &&
              hipMalloc(&v, cells * a->hd) == hipSuccess &&
              hipMalloc(&ks, cells * sizeof(float)) == hipSuccess &&
              hipMalloc(&vs, cells * sizeof(float)) == hipSuccess &&
              hipMalloc(&q, qn * sizeof(float)) == hipSuccess &&
              hipMalloc(&out, qn * sizeof(float)) == hipSuccess &&
              hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess;
    if (ok) {
        /* made-up numbers: the time of a way does not hang on them */
        const float sc = 0.01f, qv = 0.5f;
        uint32_t scb, qb;
        memcpy(&scb, &sc, 4);
        memcpy(&qb, &qv, 4);
        ok = hipMemsetAsync(k, 0x35, cells * a->hd, a->stream) == hipSuccess &&
             hipMemsetAsync(v, 0xC9, cells * a->hd, a->stream) == hipSuccess &&
             hipMemsetD32Async((hipDeviceptr_t)ks, (int)scb, cells, a->stream) == hipSuccess &&
             hipMemsetD32Async((hipDeviceptr_t)vs, (int)scb, cells, a->stream) == hipSuccess &&
             hipMemsetD32Async((hipDeviceptr_t)q, (int)qb, qn, a->stream) == hipSuccess;
    }
    for (int c = 0; ok && c < 2; c++) {
        const uint32_t n = c ? nb : 1, limit = c ? 16384 : 65536;
        uint32_t from = UINT32_MAX;
        for (uint32_t p = 1024; ok && p + n <= top && p <= limit; p *= 2) {
            janas_attn_seq s;
            memset(&s, 0, sizeof s);
            s.k = k;
            s.v = v;
            s.ks = (const float *)ks;
            s.vs = (const float *)vs;
            s.q = (const float *)q;
            s.out = (float *)out;
            s.cap = top;
            s.n = n;
            s.pos0 = p;
            const float tf = time_way(a, JANAS_ATTN_FLOAT, s, e0, e1);
            const float ti = time_way(a, JANAS_ATTN_INT16, s, e0, e1);
            if (tf < 0.0f || ti < 0.0f) {
                ok = false;
                break;
            }
            if (ti < tf) {
                if (from == UINT32_MAX)
                    from = p;
            } else {
                from = UINT32_MAX; /* it must win at every longer one */
            }
        }
        if (ok)
            a->from16[c] = from;
    }
    if (!ok) {
        /* a failed measurement leaves FLOAT, and no trace in the status */
        a->from16[0] = a->from16[1] = UINT32_MAX;
        (void)hipGetLastError();
    }
    (void)hipStreamSynchronize(a->stream);
    for (void *p : {k, v, ks, vs, q, out})
        (void)hipFree(p);
    if (e0)
        (void)hipEventDestroy(e0);
    if (e1)
        (void)hipEventDestroy(e1);
    a->scores = keep;
    a->prof = prof;
    /* the measurement's partials are not kept: back to the size before */
    if (a->part_rows > rows0) {
        (void)hipFree(a->part_ml);
        (void)hipFree(a->part_acc);
        a->part_ml = a->part_acc = nullptr;
        a->part_rows = 0;
        if (rows0 && ensure_part(a, rows0, a->stream) != JANAS_ATTN_OK)
            (void)hipGetLastError();
    }
    if (!ok)
        return;
    std::lock_guard<std::mutex> lk(g_calib_mu);
    if (!g_calib)
        g_calib = new std::vector<Calib>();
    g_calib->push_back(Calib{a->dev, a->ring, a->n_head, a->n_kv, a->hd, a->window, a->n_ctx,
                             {a->from16[0], a->from16[1]}});
    calib_save(key, a->from16);
}

/* The engine's choice for a call of n tokens at pos0 (janas_attn_run,
   attention.c:1255-1260): under AUTO over an int8 cache, measured once */
void choose_way(janas_attn *a, int kv, uint32_t n, uint32_t pos0)
{
    if (!a->scores_auto || a->kv16 || kv != kI8 || a->hd % 16)
        return;
    if (!a->calibrated)
        calibrate(a);
    a->scores = pos0 >= a->from16[n > 1] ? JANAS_ATTN_INT16 : JANAS_ATTN_FLOAT;
}

/* The same choice for a Part 2 call, of any length and any number of
   sequences: the way is measured at the first call that is not being
   captured into a graph (the measurement allocates and synchronizes) and
   is not the allocation-free entry point's (fixed); until it is measured,
   AUTO computes the FLOAT way. A call of n tokens at pos0 takes INT16 from
   from16[n > 1] on, as a call of the reference's (a prompt longer than a
   block follows the block's rule); a call of several sequences only when
   each of them would. So the way of a call never depends on what an
   earlier call was, except through the one measurement. */
void choose_way_dev(janas_attn *a, int kv, const janas_attn_seq *seqs, uint32_t n_seqs,
                    hipStream_t st, bool fixed)
{
    if (!a->scores_auto || a->kv16 || kv != kI8 || a->hd % 16)
        return;
    if (!a->calibrated && !fixed) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(st, &cs) != hipSuccess)
            (void)hipGetLastError();
        else if (cs == hipStreamCaptureStatusNone)
            calibrate(a);
    }
    bool int16 = a->calibrated != 0;
    for (uint32_t i = 0; i < n_seqs; i++)
        int16 = int16 && seqs[i].pos0 >= a->from16[seqs[i].n > 1];
    a->scores = int16 ? JANAS_ATTN_INT16 : JANAS_ATTN_FLOAT;
}

/* Key segments for a prefill sequence whose row blocks alone would leave
   compute units idle (a short prompt, a chunk of a long one): enough to
   give each unit a workgroup, at least kSegTiles key tiles each (twice as
   many with the halves' tiles, which two groups share). It depends on the
   sequence alone, so a sequence's result is the same in any launch. */
constexpr uint32_t kSegTiles = 6;

uint32_t prefill_segments(const janas_attn *a, const SeqDesc &d, bool halves, int exact)
{
    const uint64_t blocks =
        (uint64_t)a->n_kv * prefill_row_blocks(d.n, a->group, a->hd, halves, exact);
    if (blocks >= a->cus)
        return 1;
    /* the key tiles of the latest row block, which sees the most */
    const uint32_t tile = prefill_tile(a->hd, halves, exact);
    const uint32_t last = d.pos0 + d.n - 1;
    const uint32_t lo = a->window && last + 1 > a->window ? last + 1 - a->window : 0;
    const uint32_t nt = (d.end - 1) / tile - lo / tile + 1;
    const uint32_t min_tiles = halves ? 2 * kSegTiles : kSegTiles;
    uint64_t want = (a->cus + blocks - 1) / blocks;
    want = std::min<uint64_t>(want, std::max<uint32_t>(1, nt / min_tiles));
    return (uint32_t)std::min<uint64_t>(want, kMaxSegs);
}

/* Whether the prefill kernels write the Q8_K blocks with their output
   (write_out): a block is 256 / hd whole rows of one token's heads, so
   hd is 64, 128 or 256 - a whole number of rows a block, no padding - and
   the rows of a block (consecutive heads) are in one KV head's group. The
   register-staged kernel (hd 512), the exact kernel at 256 and other head
   sizes leave it to a pass over the output, unless a segment merge writes
   it. */
bool prefill_q8k_fused(const janas_attn *a)
{
    const uint32_t hd = a->hd;
    return (hd == 64 || hd == 128 || hd == 256) && a->group % (256 / hd) == 0;
}

/* Whether a prefill sequence takes the two-halves kernel (128 rows a
   workgroup as two key groups, prefill_half_kernel): f16 rows of 72..128
   numbers whose workgroups in the DMA kernel, key segments included, would
   still leave compute units idle - a prompt of about a thousand tokens, or
   an early chunk of a chunked prefill, whose key range is too short to cut
   into segments. Where segments fill the GPU the DMA kernel stays: its
   128-position tiles are cheaper a position than the halves' 64. It
   depends on the sequence alone, so a sequence's result is the same in any
   launch. */
bool prefill_halves(const janas_attn *a, int kv, const SeqDesc &d)
{
    if (!prefill_halves_supported(kv, a->hd))
        return false;
    const uint64_t wg = (uint64_t)a->n_kv * prefill_segments(a, d, false, 0) *
                        prefill_row_blocks(d.n, a->group, a->hd, false);
    return wg < a->cus;
}

/* The sequences in launches of up to kMaxSeqs, those that take the
   two-halves kernel first, then the others. exact: the sequences' k and v
   are the exact copies (run_prefill_x) of int8 (1) or int16 (2) caches;
   reserve: bytes of the fixed array they take (fixed only). */
int run_prefill_launch(janas_attn *a, int kv, int gate_mode,
                       const janas_attn_seq *seqs, uint32_t n_seqs, hipStream_t stream,
                       bool fixed, int exact = 0, uint64_t reserve = 0)
{
    for (int hv = 1; hv >= 0; hv--) {
        for (uint32_t i = 0; i < n_seqs;) {
            PrefillArgs args;
            memset(&args, 0, sizeof args);
            const janas_attn_seq *picked[kMaxSeqs];
            uint32_t m = 0, wg = 0, mg = 0;
            uint64_t rows = 0;
            for (; i < n_seqs && m < kMaxSeqs; i++) {
                SeqDesc &d = args.seq[m];
                int rc = describe(a, kv, seqs[i], d);
                if (rc)
                    return rc;
                if ((!exact && prefill_halves(a, kv, d)) != (hv == 1))
                    continue;
                d.wg0 = args.wg0s[m] = wg;
                d.mg0 = args.mg0s[m] = mg;
                d.nseg = prefill_segments(a, d, hv == 1, exact);
                d.part0 = 0;
                uint64_t nwg = (uint64_t)a->n_kv * d.nseg *
                               prefill_row_blocks(d.n, a->group, a->hd, hv == 1, exact);
                uint64_t nmg = 0;
                if (d.nseg > 1) {
                    /* partial rows from part0: (token, head) major, segment minor */
                    d.part0 = rows;
                    rows += (uint64_t)d.n * a->n_head * d.nseg;
                    nmg = pmerge_groups(d.n, a->n_head, a->hd);
                }
                if (wg + nwg > 0x7FFFFFFFu || mg + nmg > 0x7FFFFFFFu)
                    return JANAS_ATTN_ERANGE;
                wg += (uint32_t)nwg;
                mg += (uint32_t)nmg;
                picked[m++] = &seqs[i];
            }
            if (m == 0)
                break;
            Parts pt{nullptr, nullptr, fixed};
            if (rows) {
                int rc = get_parts(a, rows, stream, fixed, pt, reserve);
                if (rc)
                    return rc;
            }
            args.part_ml = pt.ml;
            args.part_acc = pt.acc;
            args.n_seqs = m;
            args.n_wg = wg;
            args.n_head = a->n_head;
            args.n_kv = a->n_kv;
            args.group = a->group;
            args.hd = a->hd;
            args.window = a->window;
            args.scale = a->scale;
            args.ring = a->ring;
            args.gate_mode = gate_mode;
            args.halves = hv;
            args.exact = exact;
            args.q8k_fused = prefill_q8k_fused(a) && !(exact && a->hd > 128);
            ProfEv *ev = fixed ? nullptr : prof_begin(a, 2, stream);
            hipError_t e = launch_prefill(kv, args, stream);
            if (e == hipSuccess && mg)
                e = launch_prefill_merge(args, mg, stream);
            prof_end(ev, stream);
            if (e != hipSuccess)
                return hip_err(e, "prefill launch");
            /* Q8_K: the kernel's output or the segment merge wrote the
               blocks, or else a pass over the output does */
            for (uint32_t j = 0; j < m; j++) {
                if (args.q8k_fused || args.seq[j].nseg > 1)
                    continue;
                int rc = put_q8k(a, picked[j], 1, stream);
                if (rc)
                    return rc;
            }
        }
    }
    return JANAS_ATTN_OK;
}

/* The exact kernel's copies (K planes, then V planes) in instance memory,
   grown on demand and ordered across streams as the partials. */
int ensure_dq(janas_attn *a, size_t bytes, hipStream_t stream)
{
    if (bytes <= a->dq_bytes)
        return JANAS_ATTN_OK;
    if (a->dq_k || a->dq_v) {
        hipError_t e = hipStreamSynchronize(stream);
        if (e == hipSuccess && a->part_stream && a->part_stream != stream)
            e = hipStreamSynchronize(a->part_stream);
        if (e != hipSuccess)
            return hip_err(e, "synchronize");
        (void)hipFree(a->dq_k);
        (void)hipFree(a->dq_v);
        a->dq_k = a->dq_v = nullptr;
        a->dq_bytes = 0;
    }
    if (hipMalloc(&a->dq_k, bytes) != hipSuccess || hipMalloc(&a->dq_v, bytes) != hipSuccess) {
        (void)hipGetLastError();
        (void)hipFree(a->dq_k);
        (void)hipFree(a->dq_v);
        a->dq_k = a->dq_v = nullptr;
        return JANAS_ATTN_ENOMEM;
    }
    a->dq_bytes = bytes;
    return JANAS_ATTN_OK;
}

/* int8 / int16 caches at head sizes up to 256 (the reference's FLOAT way,
   attention.c:107-145: the cached integers exact, f32 arithmetic): each
   sequence's visible rows - chunks c0 .. of every KV head, as the split path
   counts them - are copied as f16 planes whose sum is the integer exactly
   (launch_xcopy: linear in the positions), and prefill_exact_kernel takes
   them with the query and the weights as two f16 planes each. The copies
   live in instance memory, or, for the allocation-free entry point (fixed),
   at the start of the device's fixed array, the partials after them. */
int run_prefill_x(janas_attn *a, int kv, int gate_mode, const janas_attn_seq *seqs,
                  uint32_t n_seqs, hipStream_t stream, bool fixed)
{
    const int ex = kv == kI16 ? 2 : 1;
    for (uint32_t s0 = 0; s0 < n_seqs; s0 += kMaxSeqs) {
        const uint32_t m = std::min(kMaxSeqs, n_seqs - s0);
        XcopyArgs q[kMaxSeqs];
        size_t off[kMaxSeqs], total = 0;
        for (uint32_t i = 0; i < m; i++) {
            const janas_attn_seq &s = seqs[s0 + i];
            SeqDesc d;
            int rc = describe(a, kv, s, d);
            if (rc)
                return rc;
            memset(&q[i], 0, sizeof q[i]);
            q[i].k = s.k;
            q[i].v = s.v;
            q[i].n_kv = a->n_kv;
            q[i].cap = s.cap;
            q[i].hd = a->hd;
            q[i].ring = a->ring;
            q[i].p0 = d.c0 * kChunk;
            q[i].np = d.end - q[i].p0;
            off[i] = total;
            total += ((size_t)ex * a->n_kv * q[i].np * a->hd * sizeof(_Float16) + 255) / 256 * 256;
        }
        char *ck, *cv;
        if (fixed) {
            char *base = (char *)scratch_ptr(a->dev);
            if (!base)
                return JANAS_ATTN_EDEVICE;
            if (2 * total > JANAS_ATTN_NOALLOC_BYTES)
                return JANAS_ATTN_ERANGE;
            ck = base;
            cv = base + total;
        } else {
            int rc = ensure_dq(a, total, stream);
            if (!rc)
                rc = part_sync(a, stream);
            if (rc)
                return rc;
            ck = (char *)a->dq_k;
            cv = (char *)a->dq_v;
        }
        janas_attn_seq xs[kMaxSeqs];
        ProfEv *ev = fixed ? nullptr : prof_begin(a, 2, stream);
        for (uint32_t i = 0; i < m; i++) {
            q[i].k16 = (_Float16 *)(ck + off[i]);
            q[i].v16 = (_Float16 *)(cv + off[i]);
            hipError_t e = launch_xcopy(kv, q[i], stream);
            if (e != hipSuccess) {
                prof_end(ev, stream);
                return hip_err(e, "copy launch");
            }
            xs[i] = seqs[s0 + i];
            xs[i].k = q[i].k16;
            xs[i].v = q[i].v16;
        }
        prof_end(ev, stream);
        int rc = run_prefill_launch(a, kv, gate_mode, xs, m, stream, fixed, ex,
                                    fixed ? 2 * total : 0);
        if (rc)
            return rc;
    }
    return JANAS_ATTN_OK;
}

int run_prefill(janas_attn *a, int kv, int gate_mode,
                const janas_attn_seq *seqs, uint32_t n_seqs, hipStream_t stream,
                bool fixed = false)
{
    if (!prefill_supported(kv, a->hd))
        return JANAS_ATTN_ENOTSUP;
    if ((kv == kI8 || kv == kI16) && a->hd <= 256)
        return run_prefill_x(a, kv, gate_mode, seqs, n_seqs, stream, fixed);
    return run_prefill_launch(a, kv, gate_mode, seqs, n_seqs, stream, fixed);
}

int check_call(janas_attn *a, int kv, int gate_mode, const janas_attn_seq *seqs,
               uint32_t n_seqs)
{
    if (!a || !seqs || n_seqs == 0 || kv < kI8 || kv > kF32 ||
        gate_mode < kGateNone || gate_mode > kGateHead)
        return JANAS_ATTN_EINVAL;
    for (uint32_t i = 0; i < n_seqs; i++)
        if (gate_mode != kGateNone && !seqs[i].gate)
            return JANAS_ATTN_EINVAL;
    hipError_t e = hipSetDevice(a->dev);
    return e == hipSuccess ? JANAS_ATTN_OK : note(a, hip_err(e, "set device"));
}

[[noreturn]] void die(const char *what, int rc)
{
    fprintf(stderr, "janas_attn_run: %s (%s)\n", what,
            janas_attn_strerror(rc));
    abort();
}

}  // namespace

/* ===== Part 1 ========================================================= */

extern "C" size_t janas_attn_part_bytes(uint32_t n_head, uint32_t n_head_kv,
                                        uint32_t head_dim, uint32_t n_ctx)
{
    /* attention.c:984-992 */
    if (n_head_kv == 0)
        return 0;
    size_t chunks = (n_ctx + kChunk - 1) / kChunk;
    return (size_t)n_head_kv * chunks * JANAS_ATTN_MAX_BLOCK *
           (n_head / n_head_kv) * (head_dim + 2) * sizeof(float);
}

extern "C" struct janas_attn *janas_attn_create(uint32_t n_head,
                                                uint32_t n_head_kv,
                                                uint32_t head_dim,
                                                uint32_t n_ctx, int n_threads,
                                                int scores)
{
    /* attention.c:998-1000 */
    if (n_head_kv == 0 || n_head % n_head_kv || head_dim % 8 ||
        head_dim > 512 || n_threads < 1)
        return nullptr;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    janas_attn *a = (janas_attn *)calloc(1, sizeof(janas_attn));
    if (!a)
        return nullptr;
    a->n_head = n_head;
    a->n_kv = n_head_kv;
    a->hd = head_dim;
    a->n_ctx = n_ctx;
    a->group = n_head / n_head_kv;
    a->dev = dev;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
            hipSuccess || cus < 1) {
        (void)hipGetLastError();
        cus = 256;
    }
    a->cus = (uint32_t)cus;
    a->scale = 1.0f / sqrtf((float)head_dim);
    /* attention.c:965-982: JANAS_ATTN overrides the asked way */
    const char *e = getenv("JANAS_ATTN");
    if (e && !strcmp(e, "float"))
        scores = JANAS_ATTN_FLOAT;
    else if (e && !strcmp(e, "int16"))
        scores = JANAS_ATTN_INT16;
    else if (e && !strcmp(e, "auto"))
        scores = JANAS_ATTN_AUTO;
    a->scores_auto = scores == JANAS_ATTN_AUTO;
    /* attention.c:975-982: sixteen keys at a time, so the INT16 way needs
       head_dim a multiple of 16; AUTO takes it past 16384 positions */
    if (head_dim % 16)
        a->scores = JANAS_ATTN_FLOAT;
    else if (scores == JANAS_ATTN_FLOAT || scores == JANAS_ATTN_INT16)
        a->scores = scores;
    else
        a->scores = n_ctx > 16384 ? JANAS_ATTN_INT16 : JANAS_ATTN_FLOAT;
    a->copies = new std::vector<HostCopy>();
    a->ev_used = new std::vector<ProfEv>();
    a->ev_free = new std::vector<ProfEv>();
    a->abort_on_error = 1;
    /* the allocation-free entry point's partials on this device (a failure
       only disables that entry point) */
    (void)scratch_init(dev);
    skip_init(dev);
    /* a blocking stream: the calls that run on it (janas_attn_run, and
       Part 2 with a NULL stream) are ordered after work the caller queued
       on the legacy default stream - row writes, copies - and before what
       it queues there next */
    if (hipStreamCreateWithFlags(&a->stream, hipStreamDefault) != hipSuccess ||
        hipEventCreateWithFlags(&a->part_ev, hipEventDisableTiming) != hipSuccess) {
        (void)hipGetLastError();
        janas_attn_destroy(a);
        return nullptr;
    }
    /* the partials of a full janas_attn_run block, as the reference
       allocates them (attention.c:1013) */
    uint32_t chunks = (n_ctx + kChunk - 1) / kChunk;
    uint64_t rows = (uint64_t)n_head_kv * (chunks ? chunks : 1) *
                    JANAS_ATTN_MAX_BLOCK * a->group;
    if (ensure_part(a, rows, a->stream) != JANAS_ATTN_OK) {
        janas_attn_destroy(a);
        return nullptr;
    }
    return a;
}

extern "C" void janas_attn_destroy(struct janas_attn *a)
{
    if (!a)
        return;
    (void)hipSetDevice(a->dev);
    if (a->stream)
        (void)hipStreamSynchronize(a->stream);
    if (a->part_stream && a->part_stream != a->stream)
        (void)hipStreamSynchronize(a->part_stream);
    (void)hipFree(a->part_ml);
    (void)hipFree(a->part_acc);
    (void)hipFree(a->dq_k);
    (void)hipFree(a->dq_v);
    (void)hipFree(a->st_q);
    (void)hipFree(a->st_out);
    (void)hipFree(a->st_k);
    (void)hipFree(a->st_v);
    (void)hipFree(a->st_ks);
    (void)hipFree(a->st_vs);
    (void)hipFree(a->st_last);
    if (a->copies) {
        for (HostCopy &c : *a->copies)
            (void)hipFree(c.dev);
        delete a->copies;
    }
    (void)hipHostFree(a->pin);
    for (std::vector<ProfEv> *v : {a->ev_used, a->ev_free})
        if (v) {
            for (ProfEv &ev : *v) {
                (void)hipEventDestroy(ev.a);
                (void)hipEventDestroy(ev.b);
            }
            delete v;
        }
    if (a->part_ev)
        (void)hipEventDestroy(a->part_ev);
    if (a->stream)
        (void)hipStreamDestroy(a->stream);
    free(a);
}

extern "C" void janas_attn_set_scale(struct janas_attn *a, float scale)
{
    a->scale = scale;
}

extern "C" void janas_attn_set_window(struct janas_attn *a, uint32_t window)
{
    a->window = window;
}

extern "C" void janas_attn_set_kv16(struct janas_attn *a, int on)
{
    a->kv16 = on != 0;
    /* attention.c:1061-1066: no integer way over 16-bit keys */
    if (a->kv16 && a->scores == JANAS_ATTN_INT16)
        a->scores = JANAS_ATTN_FLOAT;
}

extern "C" void janas_attn_set_ring(struct janas_attn *a, int on)
{
    a->ring = on != 0;
}

extern "C" uint32_t janas_attn_ring_positions(uint32_t window, uint32_t n)
{
    /* attention.c:1048-1054: the window, the tokens and a chunk for the
       first token's alignment, in whole chunks */
    uint32_t need = window + n + kChunk;
    return (need + kChunk - 1) / kChunk * kChunk;
}

extern "C" void janas_attn_set_last(struct janas_attn *a, const uint32_t *last)
{
    a->last = last;
}

extern "C" int janas_attn_scores_mode(const struct janas_attn *a)
{
    return a ? a->scores : JANAS_ATTN_FLOAT;
}

extern "C" int janas_attn_scores_auto(const struct janas_attn *a)
{
    return a ? a->scores_auto : 0;
}

namespace {

/* A staging buffer of at least `need` bytes (the stream that used it is
   synchronized at the end of every janas_attn_run, so the old one is idle). */
/* the instance's pinned host buffer, at least need bytes */
bool pinned(janas_attn *a, size_t need)
{
    if (a->pin && a->pin_bytes >= need)
        return true;
    (void)hipHostFree(a->pin);
    a->pin = nullptr;
    a->pin_bytes = 0;
    if (hipHostMalloc((void **)&a->pin, need, hipHostMallocDefault) != hipSuccess) {
        (void)hipGetLastError();
        a->pin = nullptr;
        return false;
    }
    a->pin_bytes = need;
    return true;
}

bool staging(void **p, size_t *have, size_t need)
{
    if (*p && *have >= need)
        return true;
    (void)hipFree(*p);
    *p = nullptr;
    *have = 0;
    if (hipMalloc(p, need) != hipSuccess) {
        (void)hipGetLastError();
        *p = nullptr;
        return false;
    }
    *have = need;
    return true;
}

/* janas_attn_run's failure: remembered; then an abort (the default), or a
   return with a host output filled with NaN (the caller is expected to
   check janas_attn_status and recompute on its own path) */
void run_failed(janas_attn *a, const char *what, int rc, float *out, size_t qbytes,
                bool out_host)
{
    /* nothing of this call may still read or write the pinned buffer when
       the next call fills it */
    (void)hipStreamSynchronize(a->stream);
    note(a, rc);
    if (a->abort_on_error)
        die(what, rc);
    fprintf(stderr, "janas_attn_run: %s (%s)\n", what, janas_attn_strerror(rc));
    if (out && out_host) {
        const size_t nf = qbytes / sizeof(float);
        for (size_t i = 0; i < nf; i++)
            out[i] = NAN;
    }
}

}  // namespace

extern "C" void janas_attn_run(struct janas_attn *a, struct janas_pool *pool,
                               const float *q, const int8_t *k,
                               const float *ks, const int8_t *v,
                               const float *vs, uint32_t n, uint32_t pos0,
                               float *out)
{
    (void)pool;
    const uint32_t *last = a->last;
    a->last = nullptr; /* one call only (attention.c:1270-1272) */
    if (n == 0)
        return;
    const size_t hd = a->hd, cap = a->n_ctx;
    const size_t qbytes = (size_t)n * a->n_head * hd * sizeof(float);
    const bool out_host = !is_device_ptr(out);
    if (n > JANAS_ATTN_MAX_BLOCK) {
        run_failed(a, "more tokens than JANAS_ATTN_MAX_BLOCK", JANAS_ATTN_EINVAL, out, qbytes,
                   out_host);
        return;
    }
    if (hipSetDevice(a->dev) != hipSuccess) {
        (void)hipGetLastError();
        run_failed(a, "set device", JANAS_ATTN_EDEVICE, out, qbytes, out_host);
        return;
    }
    const int kv = a->kv16 ? kI16 : kI8;
    const size_t eb = elem_bytes(kv);
    uint32_t end = last ? last[n - 1] + 1 : pos0 + n;
    if (!a->ring && end > cap) {
        /* the reference reads past its cache here; a device fault is worse */
        run_failed(a, "positions past the cache", JANAS_ATTN_ERANGE, out, qbytes, out_host);
        return;
    }
    uint32_t c0 = first_chunk(a->window, pos0);
    if (a->ring && ((end + kChunk - 1) / kChunk - c0) * kChunk > cap) {
        /* attention.c:1281-1286: an abort in the reference too */
        fprintf(stderr, "janas_attn_run: %u chunks for a ring of %u\n",
                (end + kChunk - 1) / kChunk - c0, (uint32_t)(cap / kChunk));
        abort();
    }
    int rc = JANAS_ATTN_OK;
    janas_attn_seq s;
    memset(&s, 0, sizeof s);
    s.cap = a->n_ctx;
    s.n = n;
    s.pos0 = pos0;
    /* q and out: in place on the device, else through a block's buffer */
    const size_t blk_bytes =
        (size_t)JANAS_ATTN_MAX_BLOCK * a->n_head * hd * sizeof(float);
    size_t have_q = a->st_q ? blk_bytes : 0, have_out = a->st_out ? blk_bytes : 0;
    /* the cache: in place on the device, an imported copy, else the rows
       this call reads staged (the staging buffers follow the element size:
       set_kv16 may change it) */
    const size_t rows_all = (size_t)a->n_kv * cap;
    const size_t kv_bytes = rows_all * hd * eb, sc_bytes = rows_all * 4;
    struct Src {
        const void *p;
        void **st;
        size_t *have;
        size_t bytes, esz;
        const void **dst;
        const HostCopy *copy;
        bool dev;              /* device memory (asked once a call) */
    } src[4] = {{k, &a->st_k, &a->st_k_bytes, kv_bytes, hd * eb, &s.k, nullptr, false},
                {v, &a->st_v, &a->st_v_bytes, kv_bytes, hd * eb, &s.v, nullptr, false},
                {ks, (void **)&a->st_ks, &a->st_ks_bytes, sc_bytes, 4, (const void **)&s.ks,
                 nullptr, false},
                {vs, (void **)&a->st_vs, &a->st_vs_bytes, sc_bytes, 4, (const void **)&s.vs,
                 nullptr, false}};
    /* pinned memory: q, the imported caches' rows of this call's positions
       (pos0 .. end - 1, at most a ring's capacity), out */
    const bool q_host = !is_device_ptr(q);
    const size_t fresh = std::min<size_t>(end - pos0, cap);
    size_t pin_need = (q_host ? (qbytes + 15) / 16 * 16 : 0) + (out_host ? qbytes : 0);
    for (Src &x : src) {
        x.dev = is_device_ptr(x.p);
        if (!x.dev && (x.copy = find_copy(a, x.p, x.bytes)))
            pin_need += (a->n_kv * fresh * x.esz + 15) / 16 * 16;
    }
    if (pin_need && !pinned(a, pin_need)) {
        run_failed(a, "pinned host memory", JANAS_ATTN_ENOMEM, out, qbytes, out_host);
        return;
    }
    size_t pin_at = 0;
    if (!q_host) {
        s.q = q;
    } else {
        if (!staging((void **)&a->st_q, &have_q, blk_bytes)) {
            run_failed(a, "staging q", JANAS_ATTN_ENOMEM, out, qbytes, out_host);
            return;
        }
        memcpy(a->pin, q, qbytes);
        rc = hip_err(hipMemcpyAsync(a->st_q, a->pin, qbytes, hipMemcpyHostToDevice, a->stream),
                     "copy q");
        if (rc) {
            run_failed(a, "staging q", rc, out, qbytes, out_host);
            return;
        }
        pin_at = (qbytes + 15) / 16 * 16;
        s.q = a->st_q;
    }
    if (out_host) {
        if (!staging((void **)&a->st_out, &have_out, blk_bytes)) {
            run_failed(a, "staging out", JANAS_ATTN_ENOMEM, out, qbytes, out_host);
            return;
        }
        s.out = a->st_out;
    } else {
        s.out = out;
    }
    size_t r_lo = a->ring ? 0 : (size_t)c0 * kChunk;
    size_t r_hi = a->ring ? cap : end;
    RefreshArgs ra;
    memset(&ra, 0, sizeof ra);
    ra.n_kv = a->n_kv;
    ra.cap = (uint32_t)cap;
    ra.lo = (uint32_t)(a->ring ? pos0 % cap : pos0);
    ra.count = (uint32_t)fresh;
    for (Src &x : src) {
        if (x.copy) {
            /* an imported cache: its device copy, the rows of this call's
               positions taken from the host first - packed into pinned
               memory and put in place by one kernel for all four arrays,
               or by 2D copies where a row is not whole 4-byte words */
            const HostCopy *c = x.copy;
            char *dev = c->dev + ((const char *)x.p - c->host);
            if ((uintptr_t)dev % 4 || (uintptr_t)x.p % 4 || x.esz % 4) {
                rc = refresh_rows(a, dev, x.p, x.esz, pos0, end);
                if (rc) {
                    run_failed(a, "the imported cache", rc, out, qbytes, out_host);
                    return;
                }
            } else {
                char *dst = a->pin + pin_at;
                for (uint32_t h = 0; h < a->n_kv; h++) {
                    size_t lo = ra.lo, left = fresh;
                    while (left) {
                        const size_t run = std::min(left, cap - lo);
                        memcpy(dst, (const char *)x.p + ((size_t)h * cap + lo) * x.esz,
                               run * x.esz);
                        dst += run * x.esz;
                        left -= run;
                        lo = 0;
                    }
                }
                ra.src[ra.n_t] = (const uint32_t *)(a->pin + pin_at);
                ra.dst[ra.n_t] = (uint32_t *)dev;
                ra.words[ra.n_t] = (uint32_t)(x.esz / 4);
                ra.n_t++;
                pin_at += (a->n_kv * fresh * x.esz + 15) / 16 * 16;
            }
            *x.dst = dev;
            continue;
        }
        if (x.dev) {
            *x.dst = x.p;
            continue;
        }
        if (!staging(x.st, x.have, x.bytes)) {
            run_failed(a, "staging the cache", JANAS_ATTN_ENOMEM, out, qbytes, out_host);
            return;
        }
        /* per KV head, rows r_lo .. r_hi - 1 */
        size_t pitch = cap * x.esz, width = (r_hi - r_lo) * x.esz;
        const char *sp = (const char *)x.p + r_lo * x.esz;
        char *dp = (char *)*x.st + r_lo * x.esz;
        rc = hip_err(hipMemcpy2DAsync(dp, pitch, sp, pitch, width, a->n_kv,
                                      hipMemcpyHostToDevice, a->stream),
                     "copy cache rows");
        if (rc) {
            run_failed(a, "staging the cache", rc, out, qbytes, out_host);
            return;
        }
        *x.dst = *x.st;
    }
    if (last) {
        size_t have_last = a->st_last ? JANAS_ATTN_MAX_BLOCK * sizeof(uint32_t) : 0;
        if (!staging((void **)&a->st_last, &have_last, JANAS_ATTN_MAX_BLOCK * sizeof(uint32_t))) {
            run_failed(a, "staging last", JANAS_ATTN_ENOMEM, out, qbytes, out_host);
            return;
        }
        rc = hip_err(hipMemcpyAsync(a->st_last, last, n * sizeof(uint32_t),
                                    hipMemcpyHostToDevice, a->stream),
                     "copy last");
        if (rc) {
            run_failed(a, "staging last", rc, out, qbytes, out_host);
            return;
        }
        s.last = a->st_last;
        s.last_max = last[n - 1];
    }
    if (ra.n_t) {
        rc = hip_err(launch_refresh(ra, a->stream), "the imported cache's rows");
        if (rc) {
            run_failed(a, "the imported cache", rc, out, qbytes, out_host);
            return;
        }
    }
    choose_way(a, kv, n, pos0);
    rc = run_split(a, kv, kGateNone, &s, 1, a->stream);
    if (rc) {
        (void)hipStreamSynchronize(a->stream);
        run_failed(a, "attention", rc, out, qbytes, out_host);
        return;
    }
    char *pin_out = out_host ? a->pin + pin_at : nullptr;
    if (out_host) {
        rc = hip_err(hipMemcpyAsync(pin_out, a->st_out, qbytes, hipMemcpyDeviceToHost, a->stream),
                     "copy out");
        if (rc) {
            (void)hipStreamSynchronize(a->stream);
            run_failed(a, "copy out", rc, out, qbytes, out_host);
            return;
        }
    }
    rc = hip_err(hipStreamSynchronize(a->stream), "synchronize");
    if (rc) {
        run_failed(a, "synchronize", rc, out, qbytes, out_host);
        return;
    }
    if (out_host)
        memcpy(out, pin_out, qbytes);
}

extern "C" int janas_attn_status(const struct janas_attn *a)
{
    return a ? a->status : JANAS_ATTN_EINVAL;
}

extern "C" void janas_attn_clear_status(struct janas_attn *a)
{
    if (a)
        a->status = JANAS_ATTN_OK;
}

extern "C" void janas_attn_set_abort(struct janas_attn *a, int on)
{
    if (a)
        a->abort_on_error = on != 0;
}

/* The host cache's device copy: janas_cuda_import / janas_cuda_sync
   (gpu_cuda.c:372-427) - a range is copied to device memory once and found
   again by its host address. A range inside one already imported is
   already there; one that overlaps another is refused. */
extern "C" int janas_attn_import(struct janas_attn *a, const void *p, size_t bytes)
{
    if (!a || !p || bytes == 0)
        return JANAS_ATTN_EINVAL;
    if (find_copy(a, p, bytes))
        return JANAS_ATTN_OK;
    const char *q = (const char *)p;
    for (const HostCopy &c : *a->copies)
        if (q < c.host + c.bytes && c.host < q + bytes)
            return JANAS_ATTN_EINVAL;
    if (hipSetDevice(a->dev) != hipSuccess) {
        (void)hipGetLastError();
        return JANAS_ATTN_EDEVICE;
    }
    char *dev = nullptr;
    if (hipMalloc((void **)&dev, bytes) != hipSuccess) {
        (void)hipGetLastError();
        return JANAS_ATTN_ENOMEM;
    }
    int rc = hip_err(hipMemcpyAsync(dev, p, bytes, hipMemcpyHostToDevice, a->stream),
                     "import");
    if (!rc)
        rc = hip_err(hipStreamSynchronize(a->stream), "import");
    if (rc) {
        (void)hipFree(dev);
        return rc;
    }
    a->copies->push_back(HostCopy{q, bytes, dev});
    return JANAS_ATTN_OK;
}

extern "C" int janas_attn_sync(struct janas_attn *a, const void *p, size_t bytes,
                               int to_device)
{
    if (!a || !p || bytes == 0)
        return JANAS_ATTN_EINVAL;
    const HostCopy *c = find_copy(a, p, bytes);
    if (!c)
        return JANAS_ATTN_EINVAL;
    if (hipSetDevice(a->dev) != hipSuccess) {
        (void)hipGetLastError();
        return JANAS_ATTN_EDEVICE;
    }
    char *dev = c->dev + ((const char *)p - c->host);
    int rc = to_device ? hip_err(hipMemcpyAsync(dev, p, bytes, hipMemcpyHostToDevice, a->stream),
                                 "sync to the device")
                       : hip_err(hipMemcpyAsync((void *)p, dev, bytes, hipMemcpyDeviceToHost,
                                                a->stream),
                                 "sync to the host");
    if (!rc)
        rc = hip_err(hipStreamSynchronize(a->stream), "sync");
    return rc;
}

extern "C" void janas_attn_forget(struct janas_attn *a, const void *p)
{
    if (!a || !p)
        return;
    const char *q = (const char *)p;
    for (size_t i = 0; i < a->copies->size(); i++) {
        HostCopy &c = (*a->copies)[i];
        if (q >= c.host && q < c.host + c.bytes) {
            (void)hipSetDevice(a->dev);
            (void)hipStreamSynchronize(a->stream);
            (void)hipFree(c.dev);
            a->copies->erase(a->copies->begin() + i);
            return;
        }
    }
}

/* ===== Part 2 ========================================================= */

extern "C" int janas_attn_run_dev_split(struct janas_attn *a, int kv_type,
                                        int gate_mode,
                                        const struct janas_attn_seq *seqs,
                                        uint32_t n_seqs, void *stream)
{
    int rc = check_call(a, kv_type, gate_mode, seqs, n_seqs);
    if (rc)
        return rc;
    hipStream_t st = stream ? (hipStream_t)stream : a->stream;
    choose_way_dev(a, kv_type, seqs, n_seqs, st, false);
    rc = run_split(a, kv_type, gate_mode, seqs, n_seqs, st);
    return note(a, rc);
}

extern "C" int janas_attn_run_dev_prefill(struct janas_attn *a, int kv_type,
                                          int gate_mode,
                                          const struct janas_attn_seq *seqs,
                                          uint32_t n_seqs, void *stream)
{
    int rc = check_call(a, kv_type, gate_mode, seqs, n_seqs);
    if (rc)
        return rc;
    hipStream_t st = stream ? (hipStream_t)stream : a->stream;
    rc = run_prefill(a, kv_type, gate_mode, seqs, n_seqs, st);
    return note(a, rc);
}

namespace {

/* janas_attn_run_dev's routing; fixed: the partials in the device's fixed
   array (the allocation-free entry point) */
int run_dev(janas_attn *a, int kv_type, int gate_mode, const janas_attn_seq *seqs,
            uint32_t n_seqs, void *stream, bool fixed)
{
    int rc = check_call(a, kv_type, gate_mode, seqs, n_seqs);
    if (rc)
        return rc;
    hipStream_t st = stream ? (hipStream_t)stream : a->stream;
    choose_way_dev(a, kv_type, seqs, n_seqs, st, fixed);
    /* blocks of up to JANAS_ATTN_MAX_BLOCK tokens keep the split-KV
       chunking of janas_attn_run; longer prompts take the prefill tiles */
    bool any_long = false;
    for (uint32_t i = 0; i < n_seqs; i++)
        any_long |= seqs[i].n > JANAS_ATTN_MAX_BLOCK;
    /* the INT16 way is the split path's alone: an int8 cache under it
       stays there at any length */
    const bool int16 = kv_type == kI8 && a->scores == JANAS_ATTN_INT16;
    if (any_long && !int16 && prefill_supported(kv_type, a->hd)) {
        /* at most kMaxSeqs a launch: the split for short, the prefill for
           long sequences, in the caller's order within each */
        janas_attn_seq shortq[kMaxSeqs], longq[kMaxSeqs];
        for (uint32_t s0 = 0; s0 < n_seqs; s0 += kMaxSeqs) {
            const uint32_t m = std::min(kMaxSeqs, n_seqs - s0);
            uint32_t ns = 0, nl = 0;
            for (uint32_t i = 0; i < m; i++) {
                const janas_attn_seq &q = seqs[s0 + i];
                if (q.n > JANAS_ATTN_MAX_BLOCK)
                    longq[nl++] = q;
                else
                    shortq[ns++] = q;
            }
            if (ns) {
                rc = run_split(a, kv_type, gate_mode, shortq, ns, st, 3, fixed);
                if (rc)
                    return note(a, rc);
            }
            if (nl) {
                rc = run_prefill(a, kv_type, gate_mode, longq, nl, st, fixed);
                if (rc)
                    return note(a, rc);
            }
        }
    } else {
        rc = run_split(a, kv_type, gate_mode, seqs, n_seqs, st, 3, fixed);
    }
    return note(a, rc);
}

}  // namespace

extern "C" int janas_attn_run_dev(struct janas_attn *a, int kv_type,
                                  int gate_mode,
                                  const struct janas_attn_seq *seqs,
                                  uint32_t n_seqs, void *stream)
{
    return run_dev(a, kv_type, gate_mode, seqs, n_seqs, stream, false);
}

extern "C" int janas_attn_run_dev_noalloc(struct janas_attn *a, int kv_type,
                                          int gate_mode,
                                          const struct janas_attn_seq *seqs,
                                          uint32_t n_seqs, void *stream)
{
    return run_dev(a, kv_type, gate_mode, seqs, n_seqs, stream, true);
}

extern "C" int janas_attn_run_dev_kernels(struct janas_attn *a, int kv_type,
                                          int gate_mode,
                                          const struct janas_attn_seq *seqs,
                                          uint32_t n_seqs, void *stream,
                                          int kernels)
{
    int rc = check_call(a, kv_type, gate_mode, seqs, n_seqs);
    if (rc)
        return rc;
    if (kernels < 1 || kernels > 3)
        return JANAS_ATTN_EINVAL;
    return note(a, run_split(a, kv_type, gate_mode, seqs, n_seqs,
                             stream ? (hipStream_t)stream : a->stream, kernels));
}

extern "C" const char *janas_attn_strerror(int err)
{
    switch (err) {
    case JANAS_ATTN_OK:
        return "ok";
    case JANAS_ATTN_EINVAL:
        return "invalid argument";
    case JANAS_ATTN_ERANGE:
        return "positions outside the cache";
    case JANAS_ATTN_ENOMEM:
        return "out of device memory";
    case JANAS_ATTN_EDEVICE:
        return "device error";
    case JANAS_ATTN_ENOTSUP:
        return "no kernel for this element type or head size";
    }
    return "unknown error";
}

extern "C" void janas_attn_prof_enable(struct janas_attn *a, int on)
{
    a->prof = on != 0;
}

extern "C" int janas_attn_prof_read(struct janas_attn *a, uint32_t counts[3],
                                    double ms[3])
{
    for (int i = 0; i < 3; i++) {
        counts[i] = 0;
        ms[i] = 0.0;
    }
    if (hipSetDevice(a->dev) != hipSuccess)
        return JANAS_ATTN_EDEVICE;
    for (ProfEv &ev : *a->ev_used) {
        if (hipEventSynchronize(ev.b) != hipSuccess)
            return hip_err(hipGetLastError(), "event");
        float t = 0.0f;
        if (hipEventElapsedTime(&t, ev.a, ev.b) != hipSuccess)
            return hip_err(hipGetLastError(), "elapsed time");
        counts[ev.kind]++;
        ms[ev.kind] += t;
        a->ev_free->push_back(ev);
    }
    a->ev_used->clear();
    return JANAS_ATTN_OK;
}
