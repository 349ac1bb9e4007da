/*
 * Checkpoints of device tensors in the reference's formats.
 *
 * PGT1 (one tensor, core/tensor.c:604-711): "PGT1", u32 version 1, u32
 * dtype, u32 ndim, u64 shape[ndim], u64 numel, u64 elem_size, then the
 * elements row-major, all little-endian as the reference writes them on
 * x86.  PGMD (a parameter list, nn/module.c:88-185): "PGMD", u32 version 1,
 * u64 count, then one PGT1 record per parameter.  Files written here are
 * byte-identical to the reference's for the same tensors, and each side
 * reads the other's.
 *
 * The elements move between HBM and the file through two pinned host
 * buffers of 8 MiB: while one chunk is written to the file, the next is
 * copied from the device on the library stream (and the reverse on load),
 * so a checkpoint costs about max(PCIe, file) time, not their sum.  On a
 * seekable file each chunk's read is split over CK_THREADS threads (pread
 * at explicit offsets; the FILE position is moved past the data
 * afterwards): one thread's copy out of the page cache bounds a
 * single-stream load.  Saves stay one stream: writes that extend a file
 * hold its inode lock, so threaded pwrite to one file measured slower.
 * Saves are ordered after all queued device work; loads complete before
 * they return.
 */
#define _POSIX_C_SOURCE 200809L
#include "internal.h"

#include <errno.h>
#include <hip/hip_runtime_api.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <sys/types.h>
#include <unistd.h>

#define CK_CHUNK ((size_t)8 << 20)
#define CK_THREADS 4
#define CK_MIN_SLICE ((size_t)1 << 20)
#define PGT1_MAGIC "PGT1"
#define PGT1_VERSION 1u
#define PGMD_MAGIC "PGMD"
#define PGMD_VERSION 1u

static unsigned char *g_ck[2];
static hipEvent_t g_ck_ev[2];
static int g_ck_state; /* 0 = not tried, 1 = ready, -1 = failed */

static bool ck_ready(void)
{
    if (g_ck_state)
        return g_ck_state > 0;
    g_ck_state = -1;
    if (!pgd_ok())
        return false;
    for (int i = 0; i < 2; i++) {
        if (hipHostMalloc((void **)&g_ck[i], CK_CHUNK, hipHostMallocDefault) != hipSuccess ||
            hipEventCreateWithFlags(&g_ck_ev[i], hipEventDisableTiming) != hipSuccess) {
            pgd_set_err("checkpoint: cannot allocate pinned staging buffers");
            return false;
        }
    }
    g_ck_state = 1;
    return true;
}

static hipStream_t stream(void) { return (hipStream_t)pgd_stream(); }

/* one thread's share of a chunk's file read */
typedef struct {
    int fd;
    unsigned char *buf;
    size_t len;
    off_t off;
    int ok;
} ck_slice;

static void *ck_slice_run(void *arg)
{
    ck_slice *sl = arg;
    size_t done = 0;
    sl->ok = 1;
    while (done < sl->len) {
        const ssize_t r = pread(sl->fd, sl->buf + done, sl->len - done, sl->off + (off_t)done);
        if (r < 0 && errno == EINTR)
            continue;
        if (r <= 0) { /* an error, or end of file */
            sl->ok = 0;
            break;
        }
        done += (size_t)r;
    }
    return NULL;
}

/* reads [buf, buf + len) from file offset `off` in slices of at least
 * CK_MIN_SLICE, one per thread (the caller takes the first; a slice whose
 * thread cannot be started runs here too); false on any short read */
static bool ck_pread_split(int fd, unsigned char *buf, size_t len, off_t off)
{
    ck_slice sl[CK_THREADS];
    pthread_t th[CK_THREADS];
    int started[CK_THREADS] = {0};
    size_t per = (len + CK_THREADS - 1) / CK_THREADS;
    per = per < CK_MIN_SLICE ? CK_MIN_SLICE : (per + 4095) & ~(size_t)4095;
    int n = 0;
    for (size_t o = 0; o < len && n < CK_THREADS; o += per, n++)
        sl[n] = (ck_slice){fd, buf + o, len - o < per ? len - o : per, off + (off_t)o, 0};
    for (int i = 1; i < n; i++)
        started[i] = pthread_create(&th[i], NULL, ck_slice_run, &sl[i]) == 0;
    ck_slice_run(&sl[0]);
    bool ok = sl[0].ok;
    for (int i = 1; i < n; i++) {
        if (started[i])
            pthread_join(th[i], NULL);
        else
            ck_slice_run(&sl[i]);
        ok = ok && sl[i].ok;
    }
    return ok;
}

/* The file descriptor and offset for threaded reads of `nbytes` at the
 * stream's position, or -1 to use stdio (small transfers, or a stream that
 * cannot seek, such as a pipe). */
static int ck_fd(FILE *fp, size_t nbytes, off_t *base)
{
    if (nbytes < 2 * CK_MIN_SLICE || fflush(fp) != 0)
        return -1;
    const int fd = fileno(fp);
    const off_t pos = ftello(fp);
    if (fd < 0 || pos < 0 || lseek(fd, 0, SEEK_CUR) < 0)
        return -1;
    *base = pos;
    return fd;
}

bool pgc_dev_to_file(const void *dev, size_t nbytes, FILE *fp)
{
    if (!nbytes)
        return true;
    if (!ck_ready())
        return false;
    const size_t nch = (nbytes + CK_CHUNK - 1) / CK_CHUNK;
    const unsigned char *src = dev;
    for (size_t c = 0; c < nch; c++) {
        /* chunk c is in flight (queued at c - 1, or now for c = 0); queue
         * c + 1 into the other buffer, whose last chunk was written out
         * before this iteration began */
        for (size_t q = c == 0 ? 0 : c + 1; q <= c + 1 && q < nch; q++) {
            const int b = (int)(q & 1);
            const size_t off = q * CK_CHUNK, len = nbytes - off < CK_CHUNK ? nbytes - off : CK_CHUNK;
            if (hipMemcpyAsync(g_ck[b], src + off, len, hipMemcpyDeviceToHost, stream()) != hipSuccess ||
                hipEventRecord(g_ck_ev[b], stream()) != hipSuccess) {
                pgd_set_err("checkpoint: device-to-host copy failed");
                hipStreamSynchronize(stream());
                return false;
            }
        }
        const int b = (int)(c & 1);
        const size_t off = c * CK_CHUNK, len = nbytes - off < CK_CHUNK ? nbytes - off : CK_CHUNK;
        if (hipEventSynchronize(g_ck_ev[b]) != hipSuccess) {
            pgd_set_err("checkpoint: device-to-host copy failed");
            hipStreamSynchronize(stream());
            return false;
        }
        if (fwrite(g_ck[b], 1, len, fp) != len) {
            hipStreamSynchronize(stream()); /* the other buffer may still be filling */
            return false;
        }
    }
    return true;
}

bool pgc_file_to_dev(void *dev, size_t nbytes, FILE *fp)
{
    if (!nbytes)
        return true;
    if (!ck_ready())
        return false;
    const size_t nch = (nbytes + CK_CHUNK - 1) / CK_CHUNK;
    unsigned char *dst = dev;
    bool ok = true;
    off_t base = 0;
    const int fd = ck_fd(fp, nbytes, &base);
    for (size_t c = 0; c < nch && ok; c++) {
        const int b = (int)(c & 1);
        const size_t off = c * CK_CHUNK, len = nbytes - off < CK_CHUNK ? nbytes - off : CK_CHUNK;
        /* the copy out of this buffer (chunk c - 2) must be done before it
         * is refilled */
        if (c >= 2 && hipEventSynchronize(g_ck_ev[b]) != hipSuccess) {
            pgd_set_err("checkpoint: host-to-device copy failed");
            ok = false;
            break;
        }
        if (fd >= 0 ? !ck_pread_split(fd, g_ck[b], len, base + (off_t)off) : fread(g_ck[b], 1, len, fp) != len) {
            ok = false;
            break;
        }
        if (hipMemcpyAsync(dst + off, g_ck[b], len, hipMemcpyHostToDevice, stream()) != hipSuccess ||
            hipEventRecord(g_ck_ev[b], stream()) != hipSuccess) {
            pgd_set_err("checkpoint: host-to-device copy failed");
            ok = false;
        }
    }
    /* both buffers free again before returning */
    if (hipStreamSynchronize(stream()) != hipSuccess) {
        pgd_set_err("checkpoint: host-to-device copy failed");
        ok = false;
    }
    /* the stream continues after the data */
    if (ok && fd >= 0 && fseeko(fp, base + (off_t)nbytes, SEEK_SET) != 0)
        ok = false;
    return ok;
}

/* ---------------- PGT1 ---------------- */

static bool put(FILE *fp, const void *p, size_t n) { return fwrite(p, 1, n, fp) == n; }
static bool get(FILE *fp, void *p, size_t n) { return fread(p, 1, n, fp) == n; }

bool pg_tensor_save_fp(const pg_tensor *t, FILE *fp)
{
    /* tensor.c:607-650 */
    if (!t || !fp || !pgd_ok())
        return false;
    if (!t->dev && t->numel) {
        pgd_set_err("pg_tensor_save: tensor has no device storage");
        return false;
    }
    pgt_materialize((pg_tensor *)t); /* a pending zero is written as zeros */
    /* a strided view is written in logical row-major order, as the
     * reference's odometer loop writes it (tensor.c:628-647) */
    pg_tensor *own;
    const pg_tensor *src = pgt_contiguous(t, &own);
    if (!src)
        return false;
    const uint32_t ver = PGT1_VERSION, dtype = (uint32_t)t->dtype, ndim = (uint32_t)t->ndim;
    if (!put(fp, PGT1_MAGIC, 4) || !put(fp, &ver, 4) || !put(fp, &dtype, 4) || !put(fp, &ndim, 4)) {
        pg_tensor_free(own);
        return false;
    }
    for (size_t i = 0; i < t->ndim; i++) {
        const uint64_t d = (uint64_t)t->shape[i];
        if (!put(fp, &d, 8)) {
            pg_tensor_free(own);
            return false;
        }
    }
    const uint64_t numel = (uint64_t)t->numel, elem = (uint64_t)t->elem_size;
    bool ok = put(fp, &numel, 8) && put(fp, &elem, 8) && pgc_dev_to_file(src->dev, t->numel * t->elem_size, fp);
    pg_tensor_free(own);
    return ok;
}

bool pg_tensor_save(const pg_tensor *t, const char *path)
{
    if (!path)
        return false;
    FILE *fp = fopen(path, "wb");
    if (!fp)
        return false;
    bool ok = pg_tensor_save_fp(t, fp);
    return fclose(fp) == 0 && ok;
}

/* Reads and checks a PGT1 header as tensor.c:665-691 does; false on any
 * mismatch (nothing allocated). */
static bool read_header(FILE *fp, pg_dtype *dtype, size_t *ndim, size_t *shape)
{
    char magic[4];
    uint32_t ver = 0, dt = 0, nd = 0;
    if (!get(fp, magic, 4) || memcmp(magic, PGT1_MAGIC, 4) != 0)
        return false;
    if (!get(fp, &ver, 4) || ver != PGT1_VERSION)
        return false;
    if (!get(fp, &dt, 4) || !get(fp, &nd, 4))
        return false;
    if (nd == 0 || nd > PG_MAX_NDIM)
        return false;
    if (dt >= (uint32_t)PG_DTYPE_COUNT)
        return false;
    for (uint32_t i = 0; i < nd; i++) {
        uint64_t d = 0;
        if (!get(fp, &d, 8))
            return false;
        if (d == 0 || d > 10000000) /* the reference's sanity bound per dim */
            return false;
        shape[i] = (size_t)d;
    }
    uint64_t numel = 0, elem = 0;
    if (!get(fp, &numel, 8) || !get(fp, &elem, 8))
        return false;
    if (pg_shape_numel(nd, shape) != (size_t)numel)
        return false;
    if (pg_dtype_size((pg_dtype)dt) != (size_t)elem)
        return false;
    *dtype = (pg_dtype)dt;
    *ndim = nd;
    return true;
}

pg_tensor *pg_tensor_load_fp(FILE *fp)
{
    if (!fp || !pgd_ok())
        return NULL;
    pg_dtype dtype;
    size_t ndim, shape[PG_MAX_NDIM] = {0};
    if (!read_header(fp, &dtype, &ndim, shape))
        return NULL;
    pg_tensor *t = pg_tensor_empty_dtype(dtype, ndim, shape);
    if (!t)
        return NULL;
    t->pg_flags &= ~PG_TENSOR_ZERO_PENDING; /* every byte comes from the file */
    if (!pgc_file_to_dev(t->dev, t->numel * t->elem_size, fp)) {
        pg_tensor_free(t);
        return NULL;
    }
    return t;
}

pg_tensor *pg_tensor_load(const char *path)
{
    if (!path)
        return NULL;
    FILE *fp = fopen(path, "rb");
    if (!fp)
        return NULL;
    pg_tensor *t = pg_tensor_load_fp(fp);
    fclose(fp);
    return t;
}

/* ---------------- PGMD parameter lists ---------------- */

bool pg_amd_params_save_fp(pg_node *const *params, size_t n, FILE *fp)
{
    /* module.c:91-104 */
    if ((!params && n) || !fp)
        return false;
    const uint32_t ver = PGMD_VERSION;
    const uint64_t cnt = (uint64_t)n;
    if (!put(fp, PGMD_MAGIC, 4) || !put(fp, &ver, 4) || !put(fp, &cnt, 8))
        return false;
    for (size_t i = 0; i < n; i++) {
        if (!params[i] || !params[i]->value)
            return false;
        if (!pg_tensor_save_fp(params[i]->value, fp))
            return false;
    }
    return true;
}

bool pg_amd_params_save(pg_node *const *params, size_t n, const char *path)
{
    if (!path)
        return false;
    FILE *fp = fopen(path, "wb");
    if (!fp)
        return false;
    bool ok = pg_amd_params_save_fp(params, n, fp);
    return fclose(fp) == 0 && ok;
}

bool pgc_load_into(pg_tensor *dst, FILE *fp)
{
    /* a record is read whole into a new tensor, then checked against dst and
     * copied on the device: a bad record leaves dst untouched
     * (module.c:163-177) */
    pg_tensor *t = pg_tensor_load_fp(fp);
    if (!t)
        return false;
    bool same = dst && dst->numel == t->numel && dst->dtype == t->dtype && dst->ndim == t->ndim &&
                pgt_is_contiguous(dst);
    for (size_t d = 0; same && d < dst->ndim; d++)
        same = dst->shape[d] == t->shape[d];
    if (same) {
        dst->pg_flags &= ~PG_TENSOR_ZERO_PENDING;
        pgt_overwrite(dst);
        pgt_touch(dst);
        same = pgd_d2d(dst->dev, t->dev, t->numel * t->elem_size);
    }
    pg_tensor_free(t);
    return same;
}

bool pg_amd_params_load_into_fp(pg_node *const *params, size_t n, FILE *fp)
{
    /* module.c:154-180 */
    if ((!params && n) || !fp)
        return false;
    char magic[4];
    uint32_t ver = 0;
    uint64_t cnt = 0;
    if (!get(fp, magic, 4) || memcmp(magic, PGMD_MAGIC, 4) != 0)
        return false;
    if (!get(fp, &ver, 4) || ver != PGMD_VERSION)
        return false;
    if (!get(fp, &cnt, 8) || cnt != (uint64_t)n)
        return false;
    for (size_t i = 0; i < n; i++)
        if (!params[i] || !pgc_load_into(params[i]->value, fp))
            return false;
    return true;
}

bool pg_amd_params_load_into(pg_node *const *params, size_t n, const char *path)
{
    if (!path)
        return false;
    FILE *fp = fopen(path, "rb");
    if (!fp)
        return false;
    bool ok = pg_amd_params_load_into_fp(params, n, fp);
    fclose(fp);
    return ok;
}
