/* The llama.cpp bridge's calls, from C: the same header the patched ggml HIP
 * build includes (sabah-hip-bridge.h) loads libsabah_rt.so with dlopen/dlsym,
 * registers an mmap'd expert tensor by its host address, and calls
 * sabah_rt_mul_mat_id_v2 with strides computed the way ggml computes nb[]
 * (ids as a view into a wider argsort result, as llama.cpp's MoE graph builds
 * them).  A second caller passes 20 arguments, without ids_key, as the
 * reference's contract test does (tests/test_mul_mat_id_contract.py:153-154).
 *
 *   bridge_caller --load-only      load and init only; prints {"ready":..,"error":..}
 *   bridge_caller CASE_DIR         CASE_DIR/meta.txt holds
 *                                  "qt k rows n_experts n_ids n_tokens x_rows ids_ld src0_on_device";
 *                                  weights.bin, x.f32, ids.i32 the inputs; writes dst21.f32,
 *                                  dst20.f32, dst21_again.f32 and prints one JSON line.
 * Exit status 0 when every call returned what it should (the numbers are
 * compared with the oracle by the test that runs this). */
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "sabah-hip-bridge.h"

/* ggml's block size and block bytes per type (ggml type_traits). */
static int type_traits(int type, int64_t *blck, size_t *bytes) {
    switch (type) {
    case 0: case 26: *blck = 1; *bytes = 4; return 0;           /* F32, I32 */
    case 1: *blck = 1; *bytes = 2; return 0;                    /* F16 */
    case 7: *blck = 32; *bytes = 24; return 0;                  /* Q5_1 */
    case 8: *blck = 32; *bytes = 34; return 0;                  /* Q8_0 */
    case 12: *blck = 256; *bytes = 144; return 0;               /* Q4_K */
    case 13: *blck = 256; *bytes = 176; return 0;               /* Q5_K */
    case 14: *blck = 256; *bytes = 210; return 0;               /* Q6_K */
    case 18: *blck = 256; *bytes = 98; return 0;                /* IQ3_XXS */
    case 20: *blck = 32; *bytes = 18; return 0;                 /* IQ4_NL */
    case 21: *blck = 256; *bytes = 110; return 0;               /* IQ3_S */
    case 22: *blck = 256; *bytes = 82; return 0;                /* IQ2_S */
    case 23: *blck = 256; *bytes = 136; return 0;               /* IQ4_XS */
    case 42: *blck = 64; *bytes = 18; return 0;                 /* Q2_0 */
    }
    return -1;
}

/* A contiguous tensor's nb[] as ggml_new_tensor sets it. */
static int make_tensor(sabah_bridge_tensor *t, int type, int64_t ne0, int64_t ne1, int64_t ne2, void *data,
                       int is_host) {
    int64_t blck;
    size_t bytes;
    if (type_traits(type, &blck, &bytes) != 0 || ne0 % blck) return -1;
    t->type = type;
    t->ne[0] = ne0, t->ne[1] = ne1, t->ne[2] = ne2, t->ne[3] = 1;
    t->nb[0] = bytes;
    t->nb[1] = bytes * (size_t)(ne0 / blck);
    t->nb[2] = t->nb[1] * (size_t)ne1;
    t->nb[3] = t->nb[2] * (size_t)ne2;
    t->data = data;
    t->is_host = is_host;
    return 0;
}

static void *read_file(const char *dir, const char *name, size_t want) {
    char path[4096];
    snprintf(path, sizeof(path), "%s/%s", dir, name);
    FILE *f = fopen(path, "rb");
    if (!f) return NULL;
    void *p = malloc(want ? want : 1);
    const size_t got = p ? fread(p, 1, want, f) : 0;
    fclose(f);
    if (got != want) {
        free(p);
        return NULL;
    }
    return p;
}

static int write_file(const char *dir, const char *name, const void *p, size_t n) {
    char path[4096];
    snprintf(path, sizeof(path), "%s/%s", dir, name);
    FILE *f = fopen(path, "wb");
    if (!f) return -1;
    const size_t put = fwrite(p, 1, n, f);
    return fclose(f) == 0 && put == n ? 0 : -1;
}

static void json_string(const char *s) {
    putchar('"');
    for (; *s; ++s) {
        if (*s == '"' || *s == '\\') putchar('\\');
        putchar((unsigned char)*s >= 0x20 ? *s : ' ');
    }
    putchar('"');
}

static int fail_json(const char *what) {
    printf("{\"ok\": false, \"error\": ");
    json_string(what);
    printf(", \"bridge_error\": ");
    json_string(sabah_bridge_error());
    printf("}\n");
    return 1;
}

/* The 20-argument form of sabah_rt_mul_mat_id_v2: callers that predate
 * ids_key.  The library never reads that argument. */
typedef int (*mmid20_fn)(const void *, size_t, size_t, const void *, size_t, int, size_t, const void *, size_t,
                         size_t, int, int, float *, size_t, size_t, int, int, int, int, void *);

int main(int argc, char **argv) {
    if (argc != 2) {
        fprintf(stderr, "usage: %s --load-only | CASE_DIR\n", argv[0]);
        return 2;
    }
    if (strcmp(argv[1], "--load-only") == 0) {
        const int ready = sabah_bridge_load(0);
        printf("{\"ready\": %s, \"error\": ", ready ? "true" : "false");
        json_string(sabah_bridge_error());
        printf("}\n");
        return 0;
    }
    const char *dir = argv[1];
    int qt, k, rows, n_experts, n_ids, n_tokens, x_rows, ids_ld, src0_on_device;
    {
        char path[4096];
        snprintf(path, sizeof(path), "%s/meta.txt", dir);
        FILE *f = fopen(path, "r");
        if (!f || fscanf(f, "%d %d %d %d %d %d %d %d %d", &qt, &k, &rows, &n_experts, &n_ids, &n_tokens, &x_rows,
                         &ids_ld, &src0_on_device) != 9) {
            if (f) fclose(f);
            return fail_json("cannot read meta.txt");
        }
        fclose(f);
    }
    int64_t blck;
    size_t bbytes;
    if (type_traits(qt, &blck, &bbytes) != 0 || k % blck || ids_ld < n_ids || (x_rows != 1 && x_rows != n_ids))
        return fail_json("unsupported case");
    const size_t src0_bytes = bbytes * (size_t)(k / blck) * (size_t)rows * (size_t)n_experts;
    const size_t x_bytes = sizeof(float) * (size_t)k * x_rows * n_tokens;
    const size_t ids_bytes = sizeof(int32_t) * (size_t)ids_ld * n_tokens;
    const size_t dst_bytes = sizeof(float) * (size_t)rows * n_ids * n_tokens;

    if (!sabah_bridge_load(0)) return fail_json("bridge load");

    /* the expert tensor as llama.cpp holds it: an mmap of the file */
    char wpath[4096];
    snprintf(wpath, sizeof(wpath), "%s/weights.bin", dir);
    const int fd = open(wpath, O_RDONLY);
    struct stat stt;
    if (fd < 0 || fstat(fd, &stt) != 0 || (size_t)stt.st_size != src0_bytes) return fail_json("weights.bin size");
    void *mapped = mmap(NULL, src0_bytes, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (mapped == MAP_FAILED) return fail_json("mmap weights.bin");
    void *src0_data = mapped;
    if (src0_on_device) {                              /* experts offloaded by ggml itself */
        if (hipMalloc(&src0_data, src0_bytes) != hipSuccess ||
            hipMemcpy(src0_data, mapped, src0_bytes, hipMemcpyHostToDevice) != hipSuccess)
            return fail_json("device expert tensor");
    }

    void *hx = read_file(dir, "x.f32", x_bytes), *hids = read_file(dir, "ids.i32", ids_bytes);
    if (!hx || !hids) return fail_json("reading x.f32 / ids.i32");
    hipStream_t stream;                                /* ggml's backend stream */
    void *dx, *dids, *d21, *d20;
    if (hipStreamCreateWithFlags(&stream, hipStreamNonBlocking) != hipSuccess || hipMalloc(&dx, x_bytes) != hipSuccess ||
        hipMalloc(&dids, ids_bytes) != hipSuccess || hipMalloc(&d21, dst_bytes) != hipSuccess ||
        hipMalloc(&d20, dst_bytes) != hipSuccess)
        return fail_json("device buffers");
    /* Inputs and the NaN fill of the outputs go on the call's stream, which is
     * non-blocking: work on the null stream would not be ordered before the
     * calls' kernels. */
    if (hipMemcpyAsync(dx, hx, x_bytes, hipMemcpyHostToDevice, stream) != hipSuccess ||
        hipMemcpyAsync(dids, hids, ids_bytes, hipMemcpyHostToDevice, stream) != hipSuccess ||
        hipMemsetAsync(d21, 0xFF, dst_bytes, stream) != hipSuccess ||
        hipMemsetAsync(d20, 0xFF, dst_bytes, stream) != hipSuccess || hipStreamSynchronize(stream) != hipSuccess)
        return fail_json("device uploads");

    sabah_bridge_tensor src0, src1, ids, dst21, dst20;
    make_tensor(&src0, qt, k, rows, n_experts, src0_data, !src0_on_device);
    make_tensor(&src1, 0, k, x_rows, n_tokens, dx, 0);
    make_tensor(&ids, 26, ids_ld, n_tokens, 1, dids, 0);
    ids.ne[0] = n_ids;                                 /* ggml_view_2d of the first n_ids columns */
    make_tensor(&dst21, 0, rows, n_ids, n_tokens, d21, 0);
    make_tensor(&dst20, 0, rows, n_ids, n_tokens, d20, 0);

    if (sabah_bridge_mul_mat_id(&src0, &src1, &ids, &dst21, stream) != 0) return fail_json("21-argument call");
    const int banks_after_first = g_sabah_bridge.n_banks;
    const mmid20_fn call20 = (mmid20_fn)(void *)g_sabah_bridge.mul_mat_id;
    if (call20(src0.data, src0.nb[2], src0.nb[1], src1.data, src1.nb[1], (int)src1.ne[1], src1.nb[2], ids.data,
               ids.nb[0], ids.nb[1], (int)ids.ne[0], (int)ids.ne[1], (float *)dst20.data, dst20.nb[1], dst20.nb[2],
               (int)src0.ne[1], (int)src0.ne[0], (int)src0.ne[2], src0.type, (void *)stream) != 0) {
        sabah_bridge_fail("20-argument call", 1);
        return fail_json("20-argument call");
    }
    if (hipStreamSynchronize(stream) != hipSuccess) return fail_json("stream sync");
    float *h21 = (float *)malloc(dst_bytes), *h20 = (float *)malloc(dst_bytes), *hagain = (float *)malloc(dst_bytes);
    if (!h21 || !h20 || !hagain || hipMemcpyAsync(h21, d21, dst_bytes, hipMemcpyDeviceToHost, stream) != hipSuccess ||
        hipMemcpyAsync(h20, d20, dst_bytes, hipMemcpyDeviceToHost, stream) != hipSuccess ||
        hipStreamSynchronize(stream) != hipSuccess)
        return fail_json("downloads");

    /* the same op again (the next token's graph): no second upload */
    if (hipMemsetAsync(d21, 0xFF, dst_bytes, stream) != hipSuccess) return fail_json("memset");
    if (sabah_bridge_mul_mat_id(&src0, &src1, &ids, &dst21, stream) != 0) return fail_json("repeated call");
    if (hipMemcpyAsync(hagain, d21, dst_bytes, hipMemcpyDeviceToHost, stream) != hipSuccess ||
        hipStreamSynchronize(stream) != hipSuccess)
        return fail_json("repeated call download");

    /* a layout the bridge refuses: f16 activations */
    sabah_bridge_tensor half = src1;
    half.type = 1;
    half.nb[0] = 2;
    const int bad_rc = sabah_bridge_mul_mat_id(&src0, &half, &ids, &dst21, stream);
    char bad_error[512];
    snprintf(bad_error, sizeof(bad_error), "%s", sabah_bridge_error());

    if (write_file(dir, "dst21.f32", h21, dst_bytes) || write_file(dir, "dst20.f32", h20, dst_bytes) ||
        write_file(dir, "dst21_again.f32", hagain, dst_bytes))
        return fail_json("writing outputs");
    unsigned long long hits = 0, misses = 0, evictions = 0, fetched = 0, resident = 0;
    if (g_sabah_bridge.get_metrics(&hits, &misses, &evictions, &fetched, &resident) != 0)
        return fail_json("get_metrics");
    printf("{\"ok\": true, \"banks_after_first\": %d, \"banks\": %d, \"uploaded_bytes\": %llu, \"hits\": %llu, "
           "\"misses\": %llu, \"resident_bytes\": %llu, \"bad_layout_rc\": %d, \"bad_layout_error\": ",
           banks_after_first, g_sabah_bridge.n_banks, g_sabah_bridge.bytes_uploaded, hits, misses, resident, bad_rc);
    json_string(bad_error);
    printf("}\n");
    sabah_bridge_report_metrics();
    (void)hipFree(dx), (void)hipFree(dids), (void)hipFree(d21), (void)hipFree(d20);
    if (src0_on_device) (void)hipFree(src0_data);
    (void)hipStreamDestroy(stream);
    munmap(mapped, src0_bytes);
    return bad_rc == -1 ? 0 : 1;
}
