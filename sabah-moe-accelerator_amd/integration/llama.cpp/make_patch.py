"""Writes 0001-sabah-hip-mul-mat-id.patch: llama.cpp's ggml HIP build handing
MUL_MAT_ID to libsabah_rt.so.

It takes the place of the reference's patches/llama.cpp/0001-sabah-native-
mul-mat-id.patch on the same upstream base (llama.cpp 96ffdc41, the base that
patch names), at the same anchors:
  ggml-backend.cpp  the scheduler keeps a host expert tensor in the graph and
                    hands single-token MUL_MAT_IDs to the GPU backend (0001:5-56);
  ggml-cuda.cu      includes sabah-hip-bridge.h (the loader, the bank
                    registration and the call, 0001:62-206), intercepts
                    MUL_MAT_ID (0001:219-231), keeps such nodes out of HIP
                    graphs and fused kernels (0001:234-262).
The upstream lines in each hunk's context are those the reference's patch
shows; the new file's text is sabah-hip-bridge.h itself, so the patch and the
header the caller test builds cannot drift apart (a CPU test regenerates the
patch and compares).

    python make_patch.py            rewrite the patch beside this script
    python make_patch.py --check    exit 1 if the committed patch is stale
"""
from __future__ import annotations

import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
HEADER = os.path.join(HERE, "sabah-hip-bridge.h")
PATCH = os.path.join(HERE, "0001-sabah-hip-mul-mat-id.patch")

BACKEND_HUNKS = [
    (28, "", """\
 #include <sys/sysctl.h>
 #endif

+// A MUL_MAT_ID whose expert tensor stays in host memory for Sabah's library
+// (SABAH_LLAMA set): the library copies that tensor to the device once and
+// runs every later call from the copy, so the scheduler neither builds a
+// device copy of its own nor leaves small batches on the CPU.
+static bool ggml_backend_sched_sabah_host_expert(const ggml_tensor * node, const ggml_tensor * src, int src_index) {
+    static const bool enabled = std::getenv("SABAH_LLAMA") != nullptr;
+    return enabled && src_index == 0 && node->op == GGML_OP_MUL_MAT_ID && src->buffer != nullptr &&
+           ggml_backend_buffer_is_host(src->buffer) && ggml_is_quantized(src->type) && src->ne[2] > 1;
+}
+

 // backend buffer type

"""),
    (969, " static int ggml_backend_sched_backend_id_from_cur(ggml_backend_sched_t sched, st", """\
                 // check if a backend with higher prio wants to offload the op
                 if (sched->op_offload && src_backend_id == sched->n_backends - 1 && ggml_backend_buffer_is_host(src->buffer)) {
                     for (int b = 0; b < src_backend_id; b++) {
-                        if (ggml_backend_supports_op(sched->backends[b], tensor) && ggml_backend_offload_op(sched->backends[b], tensor)) {
+                        // a host expert tensor bound for Sabah's library goes to the GPU at any batch size
+                        const bool sabah = ggml_backend_sched_sabah_host_expert(tensor, src, i);
+                        if (ggml_backend_supports_op(sched->backends[b], tensor) &&
+                            (sabah || ggml_backend_offload_op(sched->backends[b], tensor))) {
                             SET_CAUSE(tensor, "1.off");
                             return b;
                         }
"""),
    (1397, " void ggml_backend_sched_split_graph(ggml_backend_sched_t sched, struct ggml_cgra", """\
                 }

                 if (src_backend_id != cur_backend_id && !ggml_backend_sched_buffer_supported(sched, src, cur_backend_id)) {
+                    if (ggml_backend_sched_sabah_host_expert(node, src, j)) {
+                        // the host tensor itself: its address is the key the library maps to its device copy
+                        tensor_id_copy(src_id, cur_backend_id, sched->cur_copy) = src;
+                        continue;
+                    }
                     // create a copy of the input in the split's backend
                     if (tensor_id_copy(src_id, cur_backend_id, 0) == NULL) {
                         ggml_backend_t backend = sched->backends[cur_backend_id];
"""),
]

CUDA_HUNKS = [
    (91, "", """\
 #include <string>
 #include <vector>

+#include "sabah-hip-bridge.h"
+
 static_assert(sizeof(half) == sizeof(ggml_fp16_t), "wrong fp16 size");

 #define GGML_LOG_WARN_ONCE(str) \\
"""),
    (137, " int ggml_cuda_get_device() {", """\
     return id;
 }

+// MUL_MAT_ID on Sabah's library (sabah-hip-bridge.h) when SABAH_LLAMA is set:
+// every expert op of a type the library decodes, whether ggml placed the
+// expert tensor in device memory or left it on the host.
+static bool ggml_cuda_sabah_type(ggml_type type) {
+    switch (type) {
+        case GGML_TYPE_Q8_0: case GGML_TYPE_Q5_1: case GGML_TYPE_Q4_K: case GGML_TYPE_Q5_K:
+        case GGML_TYPE_Q6_K: case GGML_TYPE_IQ3_XXS: case GGML_TYPE_IQ4_NL: case GGML_TYPE_IQ3_S:
+        case GGML_TYPE_IQ2_S: case GGML_TYPE_IQ4_XS: case GGML_TYPE_Q2_0:
+            return true;
+        default:
+            return false;
+    }
+}
+
+static bool ggml_cuda_sabah_owns_node(const ggml_tensor * node) {
+    static const bool enabled = std::getenv("SABAH_LLAMA") != nullptr;
+    const ggml_tensor * src0 = node->src[0];
+    return enabled && node->op == GGML_OP_MUL_MAT_ID && src0 != nullptr && src0->buffer != nullptr &&
+           ggml_cuda_sabah_type(src0->type) && src0->ne[2] > 1;
+}
+
+static sabah_bridge_tensor ggml_cuda_sabah_view(const ggml_tensor * t) {
+    sabah_bridge_tensor v;
+    v.type = (int) t->type;
+    for (int i = 0; i < 4; ++i) {
+        v.ne[i] = t->ne[i];
+        v.nb[i] = t->nb[i];
+    }
+    v.data = t->data;
+    v.is_host = t->buffer != nullptr && ggml_backend_buffer_is_host(t->buffer);
+    return v;
+}
+
+static bool ggml_cuda_sabah_mul_mat_id(ggml_backend_cuda_context & ctx, ggml_tensor * dst) {
+    if (!sabah_bridge_load(ctx.device)) {
+        GGML_LOG_ERROR("SABAH_LLAMA: %s\\n", sabah_bridge_error());
+        return false;
+    }
+    static std::once_flag report_once;
+    std::call_once(report_once, [] { std::atexit(sabah_bridge_report_metrics); });
+    const sabah_bridge_tensor src0 = ggml_cuda_sabah_view(dst->src[0]);
+    const sabah_bridge_tensor src1 = ggml_cuda_sabah_view(dst->src[1]);
+    const sabah_bridge_tensor ids  = ggml_cuda_sabah_view(dst->src[2]);
+    const sabah_bridge_tensor out  = ggml_cuda_sabah_view(dst);
+    if (sabah_bridge_mul_mat_id(&src0, &src1, &ids, &out, ctx.stream()) != 0) {
+        GGML_LOG_ERROR("SABAH_LLAMA MUL_MAT_ID: %s\\n", sabah_bridge_error());
+        return false;
+    }
+    return true;
+}
+
 static cudaError_t ggml_cuda_device_malloc(void ** ptr, size_t size, int device) {
     ggml_cuda_set_device(device);
     cudaError_t err;
"""),
    (1912, " static void ggml_cuda_mul_mat_id(ggml_backend_cuda_context & ctx, ggml_tensor *", """\
     const ggml_tensor * src1 = dst->src[1];
     const ggml_tensor * ids  = dst->src[2];

+    if (ggml_cuda_sabah_owns_node(dst)) {
+        // no other path: ggml's kernels cannot read a host expert tensor
+        if (!ggml_cuda_sabah_mul_mat_id(ctx, dst)) {
+            GGML_ABORT("SABAH_LLAMA: the MUL_MAT_ID could not run on the Sabah library");
+        }
+        return;
+    }
+
     GGML_ASSERT(src1->type == GGML_TYPE_F32);
     GGML_ASSERT(dst->type  == GGML_TYPE_F32);

"""),
    (2568, " static bool ggml_cuda_graph_check_compability(ggml_cgraph * cgraph) {", """\
         }

         // [TAG_MUL_MAT_ID_CUDA_GRAPHS]
+        // A Sabah-routed MUL_MAT_ID may copy a host expert tensor to the
+        // device or grow the library's scratch on its first call; a stream
+        // capture allows neither, so no HIP graph while such a node is present.
+        if (ggml_cuda_sabah_owns_node(node)) {
+            use_cuda_graph = false;
+        }
         if (node->op == GGML_OP_MUL_MAT_ID) {
             const int cc = ggml_cuda_info().devices[ggml_cuda_get_device()].cc;
             if (ggml_cuda_mul_mat_id_needs_sync(node, cc)) {
"""),
    (3436, " static int ggml_cuda_try_fuse(ggml_backend_cuda_context * cuda_ctx, ggml_cgraph", """\
         return 0;
     }

+    // a Sabah-routed MUL_MAT_ID must reach ggml_cuda_mul_mat_id: no fusion
+    // over it (no fusion pattern spans more than 8 nodes)
+    for (int j = i; j < cgraph->n_nodes && j < i + 8; ++j) {
+        if (ggml_cuda_sabah_owns_node(cgraph->nodes[j])) {
+            return 0;
+        }
+    }
+
     ggml_tensor * node = cgraph->nodes[i];

     if (node->op == GGML_OP_MUL) {
"""),
]


def file_diff(path: str, hunks) -> str:
    out = ["diff --git a/%s b/%s\n" % (path, path), "--- a/%s\n" % path, "+++ b/%s\n" % path]
    shift = 0
    for old_start, section, body in hunks:
        lines = [" \n" if l == "\n" else l for l in body.splitlines(keepends=True)]   # blank context lines
        assert all(l[:1] in (" ", "+", "-") for l in lines), path
        n_old = sum(1 for l in lines if l[0] in " -")
        n_new = sum(1 for l in lines if l[0] in " +")
        out.append("@@ -%d,%d +%d,%d @@%s\n" % (old_start, n_old, old_start + shift, n_new, section))
        out.extend(lines)
        shift += n_new - n_old
    return "".join(out)


def new_file_diff(path: str, text: str) -> str:
    lines = text.splitlines(keepends=True)
    assert text.endswith("\n")
    return ("diff --git a/%s b/%s\nnew file mode 100644\n--- /dev/null\n+++ b/%s\n@@ -0,0 +1,%d @@\n"
            % (path, path, path, len(lines))) + "".join("+" + l for l in lines)


def render() -> str:
    header = open(HEADER).read()
    return (file_diff("ggml/src/ggml-backend.cpp", BACKEND_HUNKS)
            + file_diff("ggml/src/ggml-cuda/ggml-cuda.cu", CUDA_HUNKS)
            + new_file_diff("ggml/src/ggml-cuda/sabah-hip-bridge.h", header))


def main(argv) -> int:
    text = render()
    if "--check" in argv:
        return 0 if os.path.exists(PATCH) and open(PATCH).read() == text else 1
    with open(PATCH, "w") as f:
        f.write(text)
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
