/* A C99 host of libmfh with no Python and no torch: what a cgo layer would
 * do through the C ABI.  It uploads FP8 codes with a scale (stored as bf16),
 * uploads two f32 vectors, runs axpyOntoResident on them, builds a graph
 * (r = relu(x * 0.5 + y)), optimises it, attaches HIP kernels, runs it as
 * Backend.CallGraph over the resident tensors and downloads every result.
 *
 * usage: c_client IN OUT
 *   IN:  int64 n_codes, int64 n, n_codes FP8 e4m3 codes, n f32 x, n f32 y
 *   OUT: the downloaded bf16 dequant (n_codes * 2 bytes), y after the axpy
 *        (n * 4 bytes) and r (n * 4 bytes)
 * Exits 1 with mfh_last_error() on the first failing call. */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include "mfh.h"
#include "mfh_backend.h"
#include "mfh_graph.h"

#define CHECK(call)                                                                 \
    do {                                                                            \
        int rc_ = (call);                                                           \
        if (rc_ != MFH_OK) {                                                        \
            fprintf(stderr, "%s failed (%d): %s\n", #call, rc_, mfh_last_error()); \
            exit(1);                                                                \
        }                                                                           \
    } while (0)

static void* read_exact(FILE* f, size_t bytes)
{
    void* p = malloc(bytes ? bytes : 1);
    if (!p || fread(p, 1, bytes, f) != bytes) {
        fprintf(stderr, "short input\n");
        exit(1);
    }
    return p;
}

static void download_to(FILE* out, mfh_backend* b, const mfh_tensor* t, size_t bytes)
{
    uint8_t dtype = 0;
    size_t got = 0;
    void* buf = malloc(bytes ? bytes : 1);
    CHECK(mfh_backend_download(b, t, &dtype, buf, bytes, &got));
    if (got != bytes || fwrite(buf, 1, bytes, out) != bytes) {
        fprintf(stderr, "download of %zu bytes gave %zu\n", bytes, got);
        exit(1);
    }
    free(buf);
}

int main(int argc, char** argv)
{
    if (argc != 3) return 2;
    FILE* in = fopen(argv[1], "rb");
    if (!in) return 2;
    int64_t n_codes = 0, n = 0;
    if (fread(&n_codes, 8, 1, in) != 1 || fread(&n, 8, 1, in) != 1) return 2;
    uint8_t* codes = read_exact(in, (size_t)n_codes);
    float* x = read_exact(in, (size_t)n * 4);
    float* y = read_exact(in, (size_t)n * 4);
    fclose(in);

    CHECK(mfh_init(0));
    mfh_backend* b = NULL;
    CHECK(mfh_backend_open(0, &b));

    /* Upload with the dequant hook: FP8 e4m3 (5) times 0.5, stored as BFloat16 (4). */
    mfh_tensor* q = NULL;
    CHECK(mfh_backend_upload_fp8(b, &n_codes, 1, 5, codes, (size_t)n_codes, 0.5f, 4, &q));

    /* Two resident f32 (2) vectors and y <- y + 0.75 x. */
    mfh_tensor* tx = NULL;
    mfh_tensor* ty = NULL;
    CHECK(mfh_backend_upload(b, &n, 1, 2, x, (size_t)n * 4, &tx));
    CHECK(mfh_backend_upload(b, &n, 1, 2, y, (size_t)n * 4, &ty));
    CHECK(mfh_axpy_onto_resident(b, ty, tx, 0.75f));

    /* r = relu(x * 0.5 + y), optimised and lowered for HIP. */
    mfh_graph* g = NULL;
    CHECK(mfh_graph_create(2, &g));
    CHECK(mfh_graph_add_input(g, "x"));
    CHECK(mfh_graph_add_input(g, "y"));
    CHECK(mfh_graph_add_node(g, "k", "math.constant", NULL, 0));
    CHECK(mfh_graph_set_attribute(g, 0, "value", 0.5));
    const char* mul_in[2] = {"x", "k"};
    const char* add_in[2] = {"a", "y"};
    const char* relu_in[1] = {"s"};
    CHECK(mfh_graph_add_node(g, "a", "math.mul", mul_in, 2));
    CHECK(mfh_graph_add_node(g, "s", "math.add", add_in, 2));
    CHECK(mfh_graph_add_node(g, "r", "activation.relu", relu_in, 1));
    CHECK(mfh_graph_set_output(g, "r", "r"));
    int32_t folded = 0;
    mfh_fusion_stats stats;
    CHECK(mfh_optimizer_run(g, 0, &folded, &stats));
    const int32_t targets[1] = {MFH_TARGET_HIP};
    int32_t attached = 0;
    CHECK(mfh_codegen_attach_kernels(g, targets, 1, 0, &attached));
    if (stats.clusters != 1 || attached != 1) {
        fprintf(stderr, "expected one fused cluster with a HIP kernel, got %d clusters, %d kernels\n",
                (int)stats.clusters, (int)attached);
        return 1;
    }
    const char* names[2] = {"x", "y"};
    const mfh_tensor* ins[2] = {tx, ty};
    const char* keys[1] = {"r"};
    mfh_tensor* outs[1] = {NULL};
    CHECK(mfh_backend_graph_call(b, g, names, ins, 2, keys, 1, outs));

    FILE* out = fopen(argv[2], "wb");
    if (!out) return 2;
    download_to(out, b, q, (size_t)n_codes * 2);
    download_to(out, b, ty, (size_t)n * 4);
    download_to(out, b, outs[0], (size_t)n * 4);
    fclose(out);

    mfh_tensor_release(outs[0]);
    mfh_tensor_release(q);
    mfh_tensor_release(tx);
    mfh_tensor_release(ty);
    mfh_graph_release(g);
    CHECK(mfh_backend_release(b));
    free(codes);
    free(x);
    free(y);
    return 0;
}
