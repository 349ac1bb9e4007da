/*
 * Device layer: one HIP device, one stream, a caching allocator.
 *
 * Every kernel and copy of the library is queued on a single non-blocking
 * stream, so a block freed on the host may be handed to the next
 * allocation at once: any later use is queued behind every earlier use.
 * Blocks are cached in size classes (powers of two up to 1 MiB, 2 MiB
 * granules above) and returned to the driver only on pg_amd_release_cached()
 * or when an allocation fails.
 */
#define _POSIX_C_SOURCE 200809L
#include "internal.h"

#include <hip/hip_runtime_api.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static hipStream_t g_stream;
static int g_init_state; /* 0 = not tried, 1 = ok, -1 = failed */
static char g_err[512];

void pgd_set_err(const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}

const char *pg_amd_last_error(void) { return g_err; }

static bool hip_ok(hipError_t e, const char *what)
{
    if (e == hipSuccess)
        return true;
    pgd_set_err("%s: %s", what, hipGetErrorString(e));
    return false;
}

bool pgd_check(int status, const char *what)
{
    if (status == 0)
        return true;
    pgd_set_err("%s: %s", what, hipGetErrorString((hipError_t)status));
    return false;
}

int pg_amd_init(void)
{
    if (g_init_state)
        return g_init_state > 0 ? 0 : -1;
    int n = 0;
    if (!hip_ok(hipGetDeviceCount(&n), "hipGetDeviceCount") || n < 1) {
        if (!g_err[0])
            pgd_set_err("no HIP device");
        g_init_state = -1;
        return -1;
    }
    if (!hip_ok(hipSetDevice(0), "hipSetDevice") ||
        !hip_ok(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking), "hipStreamCreate")) {
        g_init_state = -1;
        return -1;
    }
    /* the device address of the no-alloc workspace (pg_amd_gemm_ex_noalloc) */
    if (!pgd_check(pgk_noalloc_scratch_init(), "no-alloc workspace")) {
        g_init_state = -1;
        return -1;
    }
    g_init_state = 1;
    return 0;
}

bool pgd_initialised(void) { return g_init_state > 0; }

static int g_up_n;

bool pgd_work_pending(void) { return g_up_n > 0 || pga_lazy_pending(); }

bool pgd_ok(void) { return pg_amd_init() == 0; }

static bool up_flush(void);
static void up_flush_if_overlaps(const void *p, size_t n);

/* queues what is pending: the deferred forward ops, whose kernel either
 * performs the batched uploads itself (pgd_upload_take) or has them queued
 * first (its launch calls pgd_stream, which comes back here and queues the
 * batch while the run is flushing), then any uploads still pending */
static bool flush_pending(void)
{
    pga_lazy_flush();
    return up_flush();
}

/* A second stream for work that runs beside the main stream's: pgd_fork
 * orders it after everything queued so far, pgd_join orders everything
 * queued later on the main stream after it.  Default priority, as the
 * main stream.  Buffers the side work uses must be allocated before the
 * fork and freed after the join (the allocator's reuse is ordered on the
 * main stream). */
static hipStream_t g_side;
static hipEvent_t g_fork_ev, g_join_ev;

pgk_stream pgd_fork(void)
{
    pgk_stream main_s = pgd_stream(); /* flushes pending work first */
    if (!pgd_ok())
        return NULL;
    if (!g_side) {
        if (!hip_ok(hipStreamCreateWithFlags(&g_side, hipStreamNonBlocking), "hipStreamCreate (side)") ||
            !hip_ok(hipEventCreateWithFlags(&g_fork_ev, hipEventDisableTiming), "hipEventCreate") ||
            !hip_ok(hipEventCreateWithFlags(&g_join_ev, hipEventDisableTiming), "hipEventCreate")) {
            return NULL;
        }
    }
    if (!hip_ok(hipEventRecord(g_fork_ev, (hipStream_t)main_s), "hipEventRecord") ||
        !hip_ok(hipStreamWaitEvent(g_side, g_fork_ev, 0), "hipStreamWaitEvent"))
        return NULL;
    return (pgk_stream)g_side;
}

bool pgd_join(void)
{
    return hip_ok(hipEventRecord(g_join_ev, g_side), "hipEventRecord") &&
           hip_ok(hipStreamWaitEvent(g_stream, g_join_ev, 0), "hipStreamWaitEvent");
}

pgk_stream pgd_stream(void)
{
    /* everything queued from here on is ordered after the pending work */
    if (pg_amd_init() == 0)
        flush_pending();
    return (pgk_stream)g_stream;
}

void *pg_amd_stream(void) { return pgd_stream(); }

bool pgd_sync(void)
{
    if (!pgd_ok())
        return false;
    bool ok = flush_pending();
    return hip_ok(hipStreamSynchronize(g_stream), "hipStreamSynchronize") && ok;
}

int pg_amd_sync(void) { return pgd_sync() ? 0 : -1; }

/* ---------------- caching allocator ---------------- */

typedef struct blk {
    void *p;
    size_t cls;
    struct blk *next;
} blk;

#define NBINS 1024
static blk *g_bins[NBINS];
static size_t g_in_use, g_cached, g_cached_blocks;

static size_t size_class(size_t n)
{
    if (n <= 256)
        return 256;
    if (n <= ((size_t)1 << 20)) {
        size_t c = 512;
        while (c < n)
            c <<= 1;
        return c;
    }
    size_t g = (size_t)2 << 20;
    return (n + g - 1) / g * g;
}

static size_t bin_of(size_t cls) { return (cls / 256 * 2654435761u) % NBINS; }

static void release_all(void)
{
    if (g_init_state > 0) {
        flush_pending();
        hipStreamSynchronize(g_stream);
    }
    for (size_t i = 0; i < NBINS; i++) {
        blk *b = g_bins[i];
        while (b) {
            blk *nx = b->next;
            hipFree(b->p);
            g_cached -= b->cls;
            g_cached_blocks--;
            free(b);
            b = nx;
        }
        g_bins[i] = NULL;
    }
}

void pg_amd_release_cached(void) { release_all(); }
size_t pg_amd_bytes_in_use(void) { return g_in_use; }
size_t pg_amd_bytes_cached(void) { return g_cached; }
size_t pgd_cached_blocks(void) { return g_cached_blocks; }

void *pgd_malloc(size_t nbytes)
{
    if (!pgd_ok())
        return NULL;
    size_t cls = size_class(nbytes ? nbytes : 1);
    blk **pp = &g_bins[bin_of(cls)];
    for (blk *b = *pp; b; pp = &b->next, b = b->next) {
        if (b->cls == cls) {
            void *p = b->p;
            *pp = b->next;
            free(b);
            g_cached -= cls;
            g_cached_blocks--;
            g_in_use += cls;
            return p;
        }
    }
    void *p = NULL;
    hipError_t e = hipMalloc(&p, cls);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        release_all();
        e = hipMalloc(&p, cls);
    }
    if (!hip_ok(e, "hipMalloc"))
        return NULL;
    g_in_use += cls;
    return p;
}

void pgd_free(void *p, size_t nbytes)
{
    if (!p)
        return;
    size_t cls = size_class(nbytes ? nbytes : 1);
    up_flush_if_overlaps(p, cls);
    blk *b = malloc(sizeof *b);
    g_in_use -= cls;
    if (!b) {
        hipStreamSynchronize(g_stream);
        hipFree(p);
        return;
    }
    b->p = p;
    b->cls = cls;
    b->next = g_bins[bin_of(cls)];
    g_bins[bin_of(cls)] = b;
    g_cached += cls;
    g_cached_blocks++;
}

static void *g_scratch[PGD_SCRATCH_SLOTS];
static size_t g_scratch_n[PGD_SCRATCH_SLOTS];

void *pgd_scratch(int slot, size_t nbytes)
{
    if (slot < 0 || slot >= PGD_SCRATCH_SLOTS)
        return NULL;
    if (g_scratch_n[slot] >= nbytes && g_scratch[slot])
        return g_scratch[slot];
    if (g_scratch[slot])
        pgd_free(g_scratch[slot], g_scratch_n[slot]);
    g_scratch[slot] = pgd_malloc(nbytes);
    g_scratch_n[slot] = g_scratch[slot] ? nbytes : 0;
    return g_scratch[slot];
}

/* Host-to-device copies up to 4 MiB are batched.  The source is
 * copied into a ring of pinned staging slots that the device reads
 * directly, and the copy becomes an entry of the pending batch; one scatter
 * kernel (k_upload) writes the whole batch, launched when anything else is
 * about to be queued or waited on (pgd_stream, pgd_sync, the copies, the
 * timer, and a free of a pending destination).  So a run of leaf creations
 * costs one kernel on the compute queue instead of one DMA each, with no
 * switch between the copy engine and the compute queue.  A slot is reused
 * once the last kernel that read it has finished (its event, recorded when
 * the ring moves on from the slot).  Copies up to 4 MiB are staged as
 * slot-sized pieces, one entry each.  Larger
 * copies go straight from pageable memory, which stages them before the
 * call returns. */
#define PGD_STAGE_SLOTS 64
#define PGD_STAGE_BYTES ((size_t)256 << 10)
#define PGD_STAGE_LARGE ((size_t)4 << 20) /* staged in slot-sized pieces up to this */
static unsigned char *g_stage;     /* host address */
static unsigned char *g_stage_dev; /* the same memory as the device addresses it */
static hipEvent_t g_stage_ev[PGD_STAGE_SLOTS];
static bool g_stage_used[PGD_STAGE_SLOTS];
static int g_stage_state; /* 0 = not tried, 1 = ok, -1 = unavailable */
static int g_up_slot;
static size_t g_up_off;
static pgk_upload g_up[PGK_UPLOAD_MAX];
static bool stage_ready(void)
{
    if (g_stage_state)
        return g_stage_state > 0;
    g_stage_state = -1;
    if (hipHostMalloc((void **)&g_stage, PGD_STAGE_SLOTS * PGD_STAGE_BYTES,
                      hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess) {
        (void)hipGetLastError();
        g_stage = NULL;
        return false;
    }
    if (hipHostGetDevicePointer((void **)&g_stage_dev, g_stage, 0) != hipSuccess) {
        (void)hipGetLastError();
        hipHostFree(g_stage);
        g_stage = NULL;
        return false;
    }
    for (int i = 0; i < PGD_STAGE_SLOTS; i++) {
        if (hipEventCreateWithFlags(&g_stage_ev[i], hipEventDisableTiming) != hipSuccess) {
            (void)hipGetLastError();
            while (i-- > 0)
                hipEventDestroy(g_stage_ev[i]);
            hipHostFree(g_stage);
            g_stage = NULL;
            return false;
        }
    }
    g_stage_state = 1;
    return true;
}

/* queues the pending batch (no-op when empty) */
static bool up_flush(void)
{
    if (!g_up_n)
        return true;
    const int n = g_up_n;
    g_up_n = 0;
    return pgd_check(pgk_upload_scatter(g_up, n, (pgk_stream)g_stream), "upload");
}

int pgd_upload_take(pgk_upload *out, int max)
{
    if (!g_up_n)
        return 0;
    if (g_up_n > max)
        return -1;
    const int n = g_up_n;
    memcpy(out, g_up, (size_t)n * sizeof *out);
    g_up_n = 0;
    return n;
}

void pgd_upload_requeue(const pgk_upload *e)
{
    g_up[g_up_n++] = *e;
}

/* leaves the current slot for the next: its event is recorded behind the
 * last scatter that read it (one record per slot, not per batch), and the
 * next slot is waited for when a scatter may still read it */
static bool stage_next_slot(void)
{
    g_stage_used[g_up_slot] = hip_ok(hipEventRecord(g_stage_ev[g_up_slot], g_stream), "hipEventRecord");
    if (!g_stage_used[g_up_slot] && !hip_ok(hipStreamSynchronize(g_stream), "hipStreamSynchronize"))
        return false; /* no event to wait on later: finish now */
    g_up_slot = (g_up_slot + 1) % PGD_STAGE_SLOTS;
    if (g_stage_used[g_up_slot] && !hip_ok(hipEventSynchronize(g_stage_ev[g_up_slot]), "hipEventSynchronize"))
        return false;
    g_stage_used[g_up_slot] = false;
    return true;
}

/* a free of device memory a pending entry writes: queue the batch first,
 * so a later owner of the block is ordered after the write */
static void up_flush_if_overlaps(const void *p, size_t n)
{
    const unsigned char *a = p;
    for (int i = 0; i < g_up_n; i++) {
        const unsigned char *d = g_up[i].dst;
        if (d < a + n && a < d + g_up[i].n) {
            up_flush();
            return;
        }
    }
}

bool pgd_h2d(void *dst, const void *src, size_t nbytes)
{
    if (!nbytes)
        return true;
    if (!pgd_ok())
        return false;
    /* deferred ops recorded before this copy may read what it overwrites */
    if (pga_lazy_pending() && !flush_pending())
        return false;
    if (nbytes <= PGD_STAGE_LARGE && stage_ready()) {
        up_flush_if_overlaps(dst, nbytes); /* a second write of the same bytes keeps its order */
        /* larger copies as slot-sized pieces, each an entry of the batch */
        for (size_t done = 0; done < nbytes;) {
            const size_t piece = nbytes - done < PGD_STAGE_BYTES ? nbytes - done : PGD_STAGE_BYTES;
            size_t off = (g_up_off + 15) & ~(size_t)15;
            if (off + piece > PGD_STAGE_BYTES || g_up_n == PGK_UPLOAD_MAX) {
                if (!up_flush() || !stage_next_slot())
                    return false;
                off = 0;
            }
            const size_t at = (size_t)g_up_slot * PGD_STAGE_BYTES + off;
            memcpy(g_stage + at, (const unsigned char *)src + done, piece);
            g_up[g_up_n].dst = (unsigned char *)dst + done;
            g_up[g_up_n].src = g_stage_dev + at;
            g_up[g_up_n].n = piece;
            g_up_n++;
            g_up_off = off + piece;
            done += piece;
        }
        return true;
    }
    if (!up_flush())
        return false;
    /* pageable source: the copy is staged before the call returns */
    return hip_ok(hipMemcpyAsync(dst, src, nbytes, hipMemcpyHostToDevice, g_stream),
                  "hipMemcpyAsync H2D") &&
           hip_ok(hipStreamSynchronize(g_stream), "hipStreamSynchronize");
}

/* Small reads (a norm, a loss, one element) come back through a mapped
 * pinned buffer that the scatter kernel writes on the compute queue: no
 * copy-engine command and no staging of pageable memory sit between the
 * producing kernel and the host's wait. */
#define PGD_READ_BYTES 4096
static unsigned char *g_read, *g_read_dev;
static int g_read_state; /* 0 untried, 1 ready, -1 unavailable */

static bool read_ready(void)
{
    if (g_read_state)
        return g_read_state > 0;
    g_read_state = -1;
    if (hipHostMalloc((void **)&g_read, PGD_READ_BYTES, hipHostMallocMapped | hipHostMallocCoherent) !=
        hipSuccess) {
        (void)hipGetLastError();
        g_read = NULL;
        return false;
    }
    if (hipHostGetDevicePointer((void **)&g_read_dev, g_read, 0) != hipSuccess) {
        (void)hipGetLastError();
        hipHostFree(g_read);
        g_read = NULL;
        return false;
    }
    g_read_state = 1;
    return true;
}

bool pgd_d2h(void *dst, const void *src, size_t nbytes)
{
    if (!pgd_ok())
        return false;
    if (!nbytes)
        return pgd_sync();
    if (!flush_pending())
        return false;
    if (nbytes <= PGD_READ_BYTES && read_ready()) {
        const pgk_upload e = {g_read_dev, src, nbytes};
        if (!hip_ok((hipError_t)pgk_upload_scatter(&e, 1, (pgk_stream)g_stream), "small read") ||
            !hip_ok(hipStreamSynchronize(g_stream), "hipStreamSynchronize"))
            return false;
        memcpy(dst, g_read, nbytes);
        return true;
    }
    return hip_ok(hipMemcpyAsync(dst, src, nbytes, hipMemcpyDeviceToHost, g_stream),
                  "hipMemcpyAsync D2H") &&
           hip_ok(hipStreamSynchronize(g_stream), "hipStreamSynchronize");
}

bool pgd_d2d(void *dst, const void *src, size_t nbytes)
{
    if (!nbytes)
        return true;
    if (!pgd_ok())
        return false;
    if (!flush_pending())
        return false;
    return hip_ok(hipMemcpyAsync(dst, src, nbytes, hipMemcpyDeviceToDevice, g_stream),
                  "hipMemcpyAsync D2D");
}

/* ---------------- kernel timer ----------------
 * When enabled, hot launch sites bracket their kernels with HIP events on
 * the library stream; pg_amd_timer_read() sums the elapsed times per kind. */

typedef struct {
    hipEvent_t a, b;
    int kind;
} tev;

static tev *g_tev;
static size_t g_ntev, g_captev;
static int g_timer_on;

void pg_amd_timer_enable(int on)
{
    g_timer_on = on;
}

int pgd_tbegin(int kind)
{
    if (!g_timer_on || !pgd_ok())
        return -1;
    flush_pending();
    if (g_ntev == g_captev) {
        size_t nc = g_captev ? g_captev * 2 : 256;
        tev *p = realloc(g_tev, nc * sizeof *p);
        if (!p)
            return -1;
        g_tev = p;
        g_captev = nc;
    }
    tev *t = &g_tev[g_ntev];
    if (hipEventCreate(&t->a) != hipSuccess)
        return -1;
    if (hipEventCreate(&t->b) != hipSuccess) {
        hipEventDestroy(t->a);
        return -1;
    }
    t->kind = kind;
    hipEventRecord(t->a, g_stream);
    return (int)g_ntev++;
}

void pgd_tend(int slot)
{
    if (slot >= 0 && (size_t)slot < g_ntev)
        hipEventRecord(g_tev[slot].b, g_stream);
}

double pg_amd_timer_read(int kind, size_t *count)
{
    double total = 0.0;
    size_t n = 0;
    if (pgd_ok())
        hipStreamSynchronize(g_stream);
    for (size_t i = 0; i < g_ntev; i++) {
        if (g_tev[i].kind != kind)
            continue;
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, g_tev[i].a, g_tev[i].b) == hipSuccess) {
            total += ms;
            n++;
        }
    }
    if (count)
        *count = n;
    return total;
}

void pg_amd_timer_reset(void)
{
    if (pgd_ok())
        hipStreamSynchronize(g_stream);
    for (size_t i = 0; i < g_ntev; i++) {
        hipEventDestroy(g_tev[i].a);
        hipEventDestroy(g_tev[i].b);
    }
    g_ntev = 0;
}

double pg_amd_mfma_probe(int lds)
{
    if (!pgd_ok())
        return -1.0;
    int dev = 0, cus = 0;
    if (!hip_ok(hipGetDevice(&dev), "mfma probe") ||
        !hip_ok(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), "mfma probe") || cus < 1)
        return -1.0;
    /* one block of eight waves per CU; 8 x 4096 MFMAs per wave (~0.5 ms) */
    const int blocks = cus, iters = 4096;
    const size_t n = (size_t)blocks * 512;
    float *sink = pgd_malloc(n * sizeof(float));
    if (!sink)
        return -1.0;
    hipEvent_t a = NULL, b = NULL;
    double tflops = -1.0;
    if (hip_ok(hipEventCreate(&a), "mfma probe") && hip_ok(hipEventCreate(&b), "mfma probe") &&
        pgd_check(pgk_mfma_probe(lds ? 1 : 0, sink, n, blocks, iters, g_stream), "mfma probe") &&
        hip_ok(hipEventRecord(a, g_stream), "mfma probe") &&
        pgd_check(pgk_mfma_probe(lds ? 1 : 0, sink, n, blocks, iters, g_stream), "mfma probe") &&
        hip_ok(hipEventRecord(b, g_stream), "mfma probe") && hip_ok(hipEventSynchronize(b), "mfma probe")) {
        float ms = 0.0f;
        if (hip_ok(hipEventElapsedTime(&ms, a, b), "mfma probe") && ms > 0.0f)
            tflops = (double)blocks * 8.0 * iters * 8.0 * 32768.0 / (ms * 1e-3) / 1e12;
    }
    if (a)
        hipEventDestroy(a);
    if (b)
        hipEventDestroy(b);
    pgd_free(sink, n * sizeof(float));
    return tflops;
}
