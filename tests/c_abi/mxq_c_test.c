/* A C consumer of libmxq, compiled with gcc against include/mxq.h alone (no HIP
 * header, no C++), as a Swift or C host would use the library.
 *
 *   mxq_c_test validate
 *       argument checks and helpers that run no GPU work: status codes, messages,
 *       tiled sizes, workspace sizes, NULL / misaligned pointers, the K cap.
 *   mxq_c_test qmm FILE.safetensors PREFIX OUT_DIR
 *       loads x and the triple PREFIX.weight / .scales / .biases from the file
 *       straight into device memory (mxq_st_read), infers bits and group size
 *       from the shapes (bits = 32*wCols/K, groupSize = K/sCols, as the
 *       reference's MfLinear.load), runs mxq_quantized_matmul on the MLX layout
 *       and mxq_quantized_matmul_tiled on a tiled copy, checks that mxq_untile
 *       returns the file's bits, writes y_mlx.bin and y_tiled.bin (bf16) to
 *       OUT_DIR, and frees device memory only after synchronizing the stream.
 *
 * Prints one line per failed check and exits 1 on the first; 0 when all pass. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "mxq.h"

static int g_failed = 0;

#define CHECK(cond)                                                                    \
  do {                                                                                 \
    if (!(cond)) {                                                                     \
      fprintf(stderr, "%s:%d: check failed: %s (last error: %s)\n", __FILE__, __LINE__, \
              #cond, mxq_last_error());                                                \
      g_failed = 1;                                                                    \
      return 1;                                                                        \
    }                                                                                  \
  } while (0)

#define CALL(expr) CHECK((expr) == MXQ_OK)

static int validate(void) {
  static unsigned char arena[256] __attribute__((aligned(256)));
  void* p = arena;
  void* odd = arena + 2;
  mxq_stream s = NULL;
  void* d = arena;

  CHECK(mxq_abi_version() == MXQ_ABI_VERSION);
  CHECK(strcmp(mxq_status_string(MXQ_ERR_NULL), "MXQ_ERR_NULL") == 0);

  /* tiled sizes: row blocks x K steps x (512*bits + 256*gps) */
  CHECK(mxq_tiled_bytes(128, 4096, 64, 6) == 2 * 64 * (512 * 6 + 256));
  CHECK(mxq_tiled_bytes(100, 384, 32, 4) == 2 * 6 * (512 * 4 + 512));
  CHECK(mxq_tiled_bytes(128, 96, 32, 4) == MXQ_ERR_INVALID);
  CHECK(strstr(mxq_last_error(), "multiple of 64") != NULL);
  CHECK(mxq_tiled_bytes(128, 4096, 48, 4) == MXQ_ERR_INVALID);

  /* the workspace path: positive at large M with K % 64 == 0, zero at small M */
  CHECK(mxq_quantized_matmul_workspace_size(14400, 16384, 4096, 64, 6) > 0);
  CHECK(mxq_quantized_matmul_workspace_size(8, 16384, 4096, 64, 6) == 0);

  /* argument errors are reported before any device access */
  CHECK(mxq_quantized_matmul(p, 4, 4096, p, p, p, 64, 1, 64, 7, NULL, p, NULL) ==
        MXQ_ERR_INVALID);
  CHECK(strstr(mxq_last_error(), "bits") != NULL);
  CHECK(mxq_quantized_matmul(NULL, 4, 4096, p, p, p, 64, 1, 64, 4, NULL, p, NULL) ==
        MXQ_ERR_NULL);
  CHECK(mxq_quantized_matmul(odd, 4, 4096, p, p, p, 64, 1, 64, 4, NULL, p, NULL) ==
        MXQ_ERR_ALIGNMENT);
  CHECK(mxq_quantized_matmul(p, 4, (1ll << 22) + 64, p, p, p, 64, 1, 64, 4, NULL, p, NULL) ==
        MXQ_ERR_INVALID);
  CHECK(mxq_qmm_tiled(p, 300, 96, p, 64, 32, 4, NULL, p, NULL) == MXQ_ERR_INVALID);
  CHECK(mxq_tile_swiglu(p, p, p, 3, 64, 64, 4, p, NULL) == MXQ_ERR_INVALID);
  CHECK(mxq_untile(NULL, 64, 64, 64, 4, p, p, p, NULL) == MXQ_ERR_NULL);

  /* empty problems are no-ops */
  CALL(mxq_quantized_matmul(p, 0, 4096, p, p, p, 64, 1, 64, 4, NULL, p, NULL));
  CALL(mxq_tile(p, p, p, 0, 4096, 64, 4, p, NULL));

  /* memory and stream helpers that need no device */
  CHECK(mxq_stream_create(NULL) == MXQ_ERR_NULL);
  CHECK(mxq_malloc(NULL, 16) == MXQ_ERR_NULL);
  CALL(mxq_malloc(&d, 0));
  CHECK(d == NULL);
  CALL(mxq_free(NULL));
  CALL(mxq_stream_destroy(s));
  CALL(mxq_copy_to_device(p, p, 0, NULL));
  CHECK(mxq_copy_to_host(NULL, p, 16, NULL) == MXQ_ERR_NULL);

  /* the loader */
  mxq_safetensors* st = NULL;
  CHECK(mxq_st_open("/nonexistent/file.safetensors", &st) == MXQ_ERR_INVALID);
  CHECK(st == NULL);
  printf("validate ok\n");
  return 0;
}

/* ---- the GPU run ------------------------------------------------------------ */
typedef struct {
  void* dev;
  int64_t shape[MXQ_ST_MAX_DIMS];
  int ndim;
  int64_t nbytes;
} tensor;

static int load(mxq_safetensors* st, const char* key, const char* dtype, tensor* t,
                mxq_stream s) {
  char dt[16];
  CALL(mxq_st_info(st, key, dt, &t->ndim, t->shape, &t->nbytes));
  CHECK(strcmp(dt, dtype) == 0);
  CHECK(t->ndim == 2);
  CALL(mxq_malloc(&t->dev, (size_t)t->nbytes));
  CALL(mxq_st_read(st, key, t->dev, s));
  return 0;
}

static int write_file(const char* dir, const char* name, const void* data, size_t n) {
  char path[4096];
  snprintf(path, sizeof path, "%s/%s", dir, name);
  FILE* f = fopen(path, "wb");
  CHECK(f != NULL);
  CHECK(fwrite(data, 1, n, f) == n);
  CHECK(fclose(f) == 0);
  return 0;
}

static int qmm(const char* file, const char* prefix, const char* out_dir) {
  mxq_stream s = NULL;
  mxq_safetensors* st = NULL;
  tensor x = {0}, w = {0}, sc = {0}, bi = {0};
  char key[512];
  CALL(mxq_stream_create(&s));
  CALL(mxq_st_open(file, &st));
  CHECK(load(st, "x", "BF16", &x, s) == 0);
  snprintf(key, sizeof key, "%s.weight", prefix);
  CHECK(load(st, key, "U32", &w, s) == 0);
  snprintf(key, sizeof key, "%s.scales", prefix);
  CHECK(load(st, key, "BF16", &sc, s) == 0);
  snprintf(key, sizeof key, "%s.biases", prefix);
  CHECK(load(st, key, "BF16", &bi, s) == 0);
  CALL(mxq_stream_synchronize(s));
  mxq_st_close(st);

  const int64_t M = x.shape[0], K = x.shape[1], N = w.shape[0];
  CHECK(K > 0 && (32 * w.shape[1]) % K == 0 && K % sc.shape[1] == 0);
  const int bits = (int)(32 * w.shape[1] / K), gs = (int)(K / sc.shape[1]);
  const size_t ybytes = (size_t)(M * N) * 2;

  void *y_mlx = NULL, *y_tiled = NULL, *tiled = NULL, *w2 = NULL, *s2 = NULL, *b2 = NULL;
  CALL(mxq_malloc(&y_mlx, ybytes));
  CALL(mxq_malloc(&y_tiled, ybytes));
  CALL(mxq_quantized_matmul(x.dev, M, K, w.dev, sc.dev, bi.dev, N, 1, gs, bits, NULL, y_mlx, s));

  const int64_t tb = mxq_tiled_bytes(N, K, gs, bits);
  CHECK(tb > 0);
  CALL(mxq_malloc(&tiled, (size_t)tb));
  CALL(mxq_tile(w.dev, sc.dev, bi.dev, N, K, gs, bits, tiled, s));
  CALL(mxq_quantized_matmul_tiled(x.dev, M, K, tiled, N, gs, bits, NULL, y_tiled, s));

  /* untile returns the file's bits */
  CALL(mxq_malloc(&w2, (size_t)w.nbytes));
  CALL(mxq_malloc(&s2, (size_t)sc.nbytes));
  CALL(mxq_malloc(&b2, (size_t)bi.nbytes));
  CALL(mxq_untile(tiled, N, K, gs, bits, w2, s2, b2, s));
  unsigned char* h1 = malloc((size_t)w.nbytes);
  unsigned char* h2 = malloc((size_t)w.nbytes);
  CHECK(h1 != NULL && h2 != NULL);
  CALL(mxq_copy_to_host(h1, w.dev, (size_t)w.nbytes, s));
  CALL(mxq_copy_to_host(h2, w2, (size_t)w.nbytes, s));
  CHECK(memcmp(h1, h2, (size_t)w.nbytes) == 0);
  CALL(mxq_copy_to_host(h1, sc.dev, (size_t)sc.nbytes, s));
  CALL(mxq_copy_to_host(h2, s2, (size_t)sc.nbytes, s));
  CHECK(memcmp(h1, h2, (size_t)sc.nbytes) == 0);
  CALL(mxq_copy_to_host(h1, bi.dev, (size_t)bi.nbytes, s));
  CALL(mxq_copy_to_host(h2, b2, (size_t)bi.nbytes, s));
  CHECK(memcmp(h1, h2, (size_t)bi.nbytes) == 0);
  free(h1);
  free(h2);

  unsigned char* y = malloc(ybytes ? ybytes : 1);
  CHECK(y != NULL);
  CALL(mxq_copy_to_host(y, y_mlx, ybytes, s));
  CHECK(write_file(out_dir, "y_mlx.bin", y, ybytes) == 0);
  CALL(mxq_copy_to_host(y, y_tiled, ybytes, s));
  CHECK(write_file(out_dir, "y_tiled.bin", y, ybytes) == 0);
  free(y);

  /* device memory is released only once the stream has drained */
  CALL(mxq_stream_synchronize(s));
  void* bufs[] = {x.dev, w.dev, sc.dev, bi.dev, y_mlx, y_tiled, tiled, w2, s2, b2};
  for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; ++i) CALL(mxq_free(bufs[i]));
  CALL(mxq_stream_destroy(s));
  printf("qmm ok M=%lld K=%lld N=%lld bits=%d group_size=%d\n", (long long)M, (long long)K,
         (long long)N, bits, gs);
  return 0;
}

int main(int argc, char** argv) {
  if (argc == 2 && strcmp(argv[1], "validate") == 0) return validate() || g_failed;
  if (argc == 5 && strcmp(argv[1], "qmm") == 0) return qmm(argv[2], argv[3], argv[4]) || g_failed;
  fprintf(stderr, "usage: mxq_c_test validate | qmm FILE PREFIX OUT_DIR\n");
  return 2;
}
