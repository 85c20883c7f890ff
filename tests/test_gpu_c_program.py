"""A plain C program drives the compute entry points through the C ABI (what a
cgo / C++ shim of the reference would call): a Q4_0 tensor uploaded from host
bytes, tensor_matvec, quantize_activations_q8 and tensor_matmul_batch_v06 in
both numerics on host buffers, then the tiny model's prefill and greedy decode.
The program runs as a child process, writes its outputs to files, and they are
compared here with the oracle (bit-exact) and with the compiled reference's
golden ids."""
import os
import subprocess

import numpy as np
import pytest

from conftest import assert_bitexact, golden
from memvanta_amd import synth

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

PROGRAM = r'''
#include <stdio.h>
#include <stdlib.h>
#include "memvanta_hip.h"

static void* slurp(const char* path, size_t* n) {
    FILE* f = fopen(path, "rb");
    if (!f) return NULL;
    fseek(f, 0, SEEK_END);
    *n = (size_t)ftell(f);
    fseek(f, 0, SEEK_SET);
    void* p = malloc(*n);
    if (p && fread(p, 1, *n, f) != *n) { free(p); p = NULL; }
    fclose(f);
    return p;
}
static int spill(const char* path, const void* p, size_t n) {
    FILE* f = fopen(path, "wb");
    if (!f) return 1;
    size_t w = fwrite(p, 1, n, f);
    fclose(f);
    return w != n;
}
#define CHECK(call) do { int rc_ = (call); if (rc_ != MVH_OK) { \
    fprintf(stderr, "%s -> %d: %s\n", #call, rc_, mvh_last_error()); return 10; } } while (0)

int main(int argc, char** argv) {
    if (argc != 6) return 2;
    const char* dir = argv[1];
    const size_t rows = (size_t)atol(argv[2]), cols = (size_t)atol(argv[3]), batch = (size_t)atol(argv[4]);
    const char* gguf = argv[5];
    char path[4096];
    size_t wn = 0, xn = 0, pn = 0;
    snprintf(path, sizeof path, "%s/w.bin", dir);
    void* w = slurp(path, &wn);
    snprintf(path, sizeof path, "%s/x.bin", dir);
    float* x = (float*)slurp(path, &xn);
    snprintf(path, sizeof path, "%s/prompt.bin", dir);
    int* prompt = (int*)slurp(path, &pn);
    if (!w || !x || !prompt || xn != batch * cols * sizeof(float)) return 3;

    mvh_context* ctx = NULL;
    mvh_tensor* t = NULL;
    CHECK(mvh_context_create(0, &ctx));
    CHECK(mvh_tensor_upload(ctx, "blk.0.ffn_up.weight", MVH_TYPE_Q4_0, cols, rows, w, wn, &t));
    float* y = (float*)malloc(rows * sizeof(float));
    float* yb = (float*)malloc(batch * rows * sizeof(float));
    int8_t* q = (int8_t*)malloc(batch * cols);
    float* d = (float*)malloc(batch * cols / 32 * sizeof(float));
    CHECK(mvh_matvec(ctx, t, x, y, MVH_HOST));
    snprintf(path, sizeof path, "%s/matvec.bin", dir);
    if (spill(path, y, rows * sizeof(float))) return 4;
    CHECK(mvh_quantize_q8(ctx, x, batch, cols, q, d, MVH_HOST));
    snprintf(path, sizeof path, "%s/q.bin", dir);
    if (spill(path, q, batch * cols)) return 4;
    snprintf(path, sizeof path, "%s/d.bin", dir);
    if (spill(path, d, batch * cols / 32 * sizeof(float))) return 4;
    CHECK(mvh_matmul_batch_v06(ctx, t, x, yb, batch, MVH_ACT_Q8, MVH_HOST));
    snprintf(path, sizeof path, "%s/v06_q8.bin", dir);
    if (spill(path, yb, batch * rows * sizeof(float))) return 4;
    CHECK(mvh_matmul_batch_v06(ctx, t, x, yb, batch, MVH_ACT_REF, MVH_HOST));
    snprintf(path, sizeof path, "%s/v06_ref.bin", dir);
    if (spill(path, yb, batch * rows * sizeof(float))) return 4;
    CHECK(mvh_tensor_free(t));
    CHECK(mvh_context_destroy(ctx));

    mvh_model* m = NULL;
    int ids[12];
    size_t pos = 0;
    CHECK(mvh_model_open(gguf, 0, 256, 128, MVH_KV_F16, MVH_ACT_Q8, 32, &m));
    CHECK(mvh_model_prefill(m, prompt, pn / sizeof(int), 32, NULL));
    CHECK(mvh_model_generate_greedy(m, 17, 12, ids, NULL));
    CHECK(mvh_model_position(m, &pos));
    CHECK(mvh_model_close(m));
    snprintf(path, sizeof path, "%s/ids.bin", dir);
    if (spill(path, ids, sizeof ids)) return 4;
    printf("ok %zu\n", pos);
    return 0;
}
'''


def test_c_program_compute_calls_match_oracle(tmp_path, oracle):
    rng = np.random.default_rng(321)
    rows, cols, batch = 300, 4096, 5
    w = synth.quantize_q4_0(rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02))
    x = synth.activations(rng, batch, cols)
    g = golden("model_tiny.npz")
    gguf = str(tmp_path / "tiny.gguf")
    assert synth.write_model(synth.TINY, gguf, seed=1234) == str(g["model_sha"])
    w.tofile(tmp_path / "w.bin")
    np.ascontiguousarray(x, np.float32).tofile(tmp_path / "x.bin")
    np.asarray(g["prompt"], np.int32).tofile(tmp_path / "prompt.bin")

    src = tmp_path / "drive_abi.c"
    src.write_text(PROGRAM)
    exe = tmp_path / "drive_abi"
    lib_dir = os.path.join(ROOT, "memvanta_amd")
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"), str(src), "-o",
                    str(exe), "-L", lib_dir, "-lmemvanta_hip", "-Wl,-rpath," + lib_dir], check=True)
    run = subprocess.run([str(exe), str(tmp_path), str(rows), str(cols), str(batch), gguf], capture_output=True,
                         text=True, timeout=120)
    assert run.returncode == 0, run.stderr
    assert run.stdout.split() == ["ok", str(len(g["prompt"]) + 12)]

    def load(name, dt):
        return np.fromfile(tmp_path / name, dtype=dt)

    assert_bitexact(load("matvec.bin", np.float32), oracle.matvec(w, synth.Q4_0, rows, cols, x[0]), "matvec")
    q, d = load("q.bin", np.int8).reshape(batch, cols), load("d.bin", np.float32).reshape(batch, cols // 32)
    for b in range(batch):
        q_ref, d_ref = oracle.quantize_q8(x[b])
        assert np.array_equal(q[b], q_ref)
        assert_bitexact(d[b], d_ref, f"Q8 scales of row {b}")
    for name, force in (("v06_q8.bin", True), ("v06_ref.bin", False)):
        want = oracle.matmul_batch_v06(w, synth.Q4_0, rows, cols, x, is_ffn=True, force_q8=force)
        assert_bitexact(load(name, np.float32).reshape(batch, rows), want.reshape(batch, rows), name)
    assert load("ids.bin", np.int32).tolist() == g["decode_ids_m1"].tolist()
