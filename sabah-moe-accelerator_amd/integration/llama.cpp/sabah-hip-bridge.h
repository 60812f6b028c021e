/* sabah-hip-bridge.h: ggml's HIP build handing MUL_MAT_ID to libsabah_rt.so.
 *
 * The caller side of the boundary (the llama.cpp bridge of the reference,
 * patches/llama.cpp/0001-sabah-native-mul-mat-id.patch:138-206), restated for
 * an HBM-resident expert bank:
 *   - the loader opens the library named by SABAH_RT_LIB (default
 *     libsabah_rt.so) and resolves sabah_rt_init, sabah_rt_mul_mat_id_v2,
 *     sabah_rt_last_error, sabah_rt_get_metrics (0001:138-175) and
 *     sabah_rt_register_bank;
 *   - an expert tensor ggml left in host memory (--cpu-moe, or an mmap'd
 *     GGUF) is copied to the device once, on its first MUL_MAT_ID, and
 *     registered under its host address, so every later call passes that
 *     address and the library maps it to the device copy; an expert tensor
 *     ggml already placed in device memory is passed as it is;
 *   - the call hands over ggml's own byte strides (nb[]) and extents (ne[])
 *     unchanged (0001:193-200) on the backend's stream.
 *
 * Plain C, and valid C++: ggml-cuda.cu includes it in the patched HIP build,
 * and the caller test (tests/bridge/bridge_caller.c) drives the same code
 * from C.  The bridge sees tensors through sabah_bridge_tensor, the parts of
 * a ggml_tensor the call reads, filled by the including file. */
#pragma once

#include <dlfcn.h>
#include <limits.h>
#include <pthread.h>
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#define SABAH_BRIDGE_TYPE_F32 0   /* GGML_TYPE_F32 */
#define SABAH_BRIDGE_TYPE_I32 26  /* GGML_TYPE_I32 */
#define SABAH_BRIDGE_MAX_BANKS 4096

typedef struct sabah_bridge_tensor {
    int type;           /* ggml_type */
    int64_t ne[4];      /* extents, ggml order (ne[0] innermost) */
    size_t nb[4];       /* byte strides */
    void *data;
    int is_host;        /* ggml_backend_buffer_is_host(tensor->buffer) */
} sabah_bridge_tensor;

typedef int (*sabah_bridge_init_fn)(int);
typedef int (*sabah_bridge_mmid_fn)(const void *, size_t, size_t,
                                    const void *, size_t, int, size_t,
                                    const void *, size_t, size_t, int, int,
                                    float *, size_t, size_t,
                                    int, int, int, int, void *, const void *);
typedef const char *(*sabah_bridge_last_error_fn)(void);
typedef int (*sabah_bridge_metrics_fn)(unsigned long long *, unsigned long long *, unsigned long long *,
                                       unsigned long long *, unsigned long long *);
typedef int (*sabah_bridge_register_fn)(const void *, void *, size_t, size_t, int);

typedef struct sabah_bridge_state {
    void *handle;
    int ready;
    sabah_bridge_init_fn init;
    sabah_bridge_mmid_fn mul_mat_id;
    sabah_bridge_last_error_fn last_error;
    sabah_bridge_metrics_fn get_metrics;
    sabah_bridge_register_fn register_bank;
    char error[512];
    pthread_mutex_t banks_mu;
    int n_banks;
    const void *bank_keys[SABAH_BRIDGE_MAX_BANKS];  /* host tensors already copied and registered */
    void *bank_dev[SABAH_BRIDGE_MAX_BANKS];
    unsigned long long bytes_uploaded;
} sabah_bridge_state;

static sabah_bridge_state g_sabah_bridge = {NULL, 0, NULL, NULL, NULL, NULL, NULL, {0},
                                            PTHREAD_MUTEX_INITIALIZER, 0, {NULL}, {NULL}, 0};
static pthread_once_t g_sabah_bridge_once = PTHREAD_ONCE_INIT;
static int g_sabah_bridge_device = 0;

/* The message of the last bridge failure: the library's own message where
 * the library failed. */
static const char *sabah_bridge_error(void) { return g_sabah_bridge.error; }

static void sabah_bridge_fail(const char *what, int from_library) {
    sabah_bridge_state *b = &g_sabah_bridge;
    if (from_library && b->last_error)
        snprintf(b->error, sizeof(b->error), "%s: %s", what, b->last_error());
    else
        snprintf(b->error, sizeof(b->error), "%s", what);
}

static void sabah_bridge_load_once(void) {
    sabah_bridge_state *b = &g_sabah_bridge;
    const char *configured = getenv("SABAH_RT_LIB");
    const char *path = configured && *configured ? configured : "libsabah_rt.so";
    b->handle = dlopen(path, RTLD_NOW | RTLD_LOCAL);
    if (!b->handle) {
        snprintf(b->error, sizeof(b->error), "Sabah runtime could not be loaded: %s (%s)", path, dlerror());
        return;
    }
    b->init = (sabah_bridge_init_fn)dlsym(b->handle, "sabah_rt_init");
    b->mul_mat_id = (sabah_bridge_mmid_fn)dlsym(b->handle, "sabah_rt_mul_mat_id_v2");
    b->last_error = (sabah_bridge_last_error_fn)dlsym(b->handle, "sabah_rt_last_error");
    b->get_metrics = (sabah_bridge_metrics_fn)dlsym(b->handle, "sabah_rt_get_metrics");
    b->register_bank = (sabah_bridge_register_fn)dlsym(b->handle, "sabah_rt_register_bank");
    if (!b->init || !b->mul_mat_id || !b->last_error || !b->get_metrics || !b->register_bank) {
        snprintf(b->error, sizeof(b->error), "%s is missing the native MUL_MAT_ID ABI", path);
        return;
    }
    if (b->init(g_sabah_bridge_device) != 0) {
        sabah_bridge_fail("Sabah runtime init failed", 1);
        return;
    }
    b->ready = 1;
}

/* Opens and initialises the library on `device` the first time it is called
 * (later calls return the first call's outcome).  Returns 1 when ready. */
static int sabah_bridge_load(int device) {
    g_sabah_bridge_device = device;
    pthread_once(&g_sabah_bridge_once, sabah_bridge_load_once);
    return g_sabah_bridge.ready;
}

/* The device copy of a host expert tensor: made and registered on first
 * sight, looked up afterwards.  The copy is issued on the call's stream and
 * waited for there, so it is complete, in that stream's order, before the
 * call's kernels read it (ggml's stream is non-blocking: a copy on the null
 * stream would not be ordered before them).  Returns 0, or -1 with the bridge
 * error set. */
static int sabah_bridge_register_host(const sabah_bridge_tensor *src0, hipStream_t stream) {
    sabah_bridge_state *b = &g_sabah_bridge;
    const size_t bytes = src0->nb[2] * (size_t)src0->ne[2];
    int rc = 0;
    pthread_mutex_lock(&b->banks_mu);
    for (int i = 0; i < b->n_banks; ++i)
        if (b->bank_keys[i] == src0->data) {
            pthread_mutex_unlock(&b->banks_mu);
            return 0;
        }
    void *dev = NULL;
    if (b->n_banks == SABAH_BRIDGE_MAX_BANKS) {
        sabah_bridge_fail("too many host expert tensors for the bridge's bank table", 0);
        rc = -1;
    } else if (hipMalloc(&dev, bytes) != hipSuccess) {
        snprintf(b->error, sizeof(b->error), "no device memory for a %zu-byte expert tensor", bytes);
        rc = -1;
    } else if (hipMemcpyAsync(dev, src0->data, bytes, hipMemcpyHostToDevice, stream) != hipSuccess ||
               hipStreamSynchronize(stream) != hipSuccess) {
        snprintf(b->error, sizeof(b->error), "copying a %zu-byte expert tensor to the device failed", bytes);
        (void)hipFree(dev);
        rc = -1;
    } else if (b->register_bank(src0->data, dev, bytes, src0->nb[2], (int)src0->ne[2]) != 0) {
        sabah_bridge_fail("registering an expert tensor failed", 1);
        (void)hipFree(dev);
        rc = -1;
    } else {
        b->bank_keys[b->n_banks] = src0->data;
        b->bank_dev[b->n_banks] = dev;
        ++b->n_banks;
        b->bytes_uploaded += bytes;
    }
    pthread_mutex_unlock(&b->banks_mu);
    return rc;
}

/* dst = MUL_MAT_ID(src0, src1, ids) on `stream`, ggml's argument meaning:
 * src0 [k, rows, n_experts] quantized, src1 [k, 1 or n_ids, n_tokens] f32,
 * ids [n_ids, n_tokens] i32, dst [rows, n_ids, n_tokens] f32.  Returns 0, or
 * -1 with sabah_bridge_error() set; the caller aborts on -1, as a Sabah-routed
 * op has no other path (0001:223-229). */
static int sabah_bridge_mul_mat_id(const sabah_bridge_tensor *src0, const sabah_bridge_tensor *src1,
                                   const sabah_bridge_tensor *ids, const sabah_bridge_tensor *dst,
                                   hipStream_t stream) {
    sabah_bridge_state *b = &g_sabah_bridge;
    if (!b->ready) return -1;
    if (src1->type != SABAH_BRIDGE_TYPE_F32 || dst->type != SABAH_BRIDGE_TYPE_F32 ||
        src1->nb[0] != sizeof(float) || dst->nb[0] != sizeof(float) || ids->type != SABAH_BRIDGE_TYPE_I32 ||
        src0->ne[3] != 1 || src1->ne[3] != 1 || ids->ne[2] != 1 || dst->ne[3] != 1 ||
        src1->ne[1] > INT_MAX || src0->ne[0] > INT_MAX || src0->ne[1] > INT_MAX || src0->ne[2] > INT_MAX ||
        ids->ne[0] > INT_MAX || ids->ne[1] > INT_MAX) {
        sabah_bridge_fail("unsupported MUL_MAT_ID layout", 0);
        return -1;
    }
    if (src0->is_host && sabah_bridge_register_host(src0, stream) != 0) return -1;
    const int rc = b->mul_mat_id(src0->data, src0->nb[2], src0->nb[1],
                                 src1->data, src1->nb[1], (int)src1->ne[1], src1->nb[2],
                                 ids->data, ids->nb[0], ids->nb[1], (int)ids->ne[0], (int)ids->ne[1],
                                 (float *)dst->data, dst->nb[1], dst->nb[2],
                                 (int)src0->ne[1], (int)src0->ne[0], (int)src0->ne[2], src0->type,
                                 (void *)stream, ids->data);   /* ids_key: ignored by this library */
    if (rc != 0) {
        sabah_bridge_fail("MUL_MAT_ID failed", 1);
        return -1;
    }
    return 0;
}

/* One line of the library's counters on stderr when SABAH_LLAMA_TRACE is
 * set, for an atexit hook (0001:112-128). */
static void sabah_bridge_report_metrics(void) {
    sabah_bridge_state *b = &g_sabah_bridge;
    if (!b->ready || !getenv("SABAH_LLAMA_TRACE")) return;
    unsigned long long hits = 0, misses = 0, evictions = 0, fetched = 0, resident = 0;
    if (b->get_metrics(&hits, &misses, &evictions, &fetched, &resident) == 0)
        fprintf(stderr, "SABAH_LLAMA metrics: hits=%llu misses=%llu evictions=%llu fetched_bytes=%llu "
                        "resident_bytes=%llu uploaded_bytes=%llu banks=%d\n",
                hits, misses, evictions, fetched, resident, b->bytes_uploaded, b->n_banks);
}
