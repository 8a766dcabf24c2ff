// Host-side exercise of libsfgemm's C ABI for the sanitizer build (see
// tests/test_sanitize_cpu.py): argument validation, the kernel planner
// over many shapes, the no-allocation entry point's scratch check, error
// texts and the runtime wrappers' failure paths, all without a GPU.  Built
// with AddressSanitizer and UndefinedBehaviorSanitizer on the host code;
// any report makes the process fail.  Exits 0 when every expectation holds.
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "sfgemm.h"

static int g_bad = 0;
#define EXPECT(cond)                                                         \
  do {                                                                       \
    if (!(cond)) {                                                           \
      fprintf(stderr, "%s:%d: expectation failed: %s (last error: %s)\n",    \
              __FILE__, __LINE__, #cond, sf_last_error());                   \
      ++g_bad;                                                               \
    }                                                                        \
  } while (0)

static void* P(uintptr_t v) { return (void*)v; }

int main() {
  // status texts, version, empty last error
  for (int s = -6; s <= 0; ++s) EXPECT(sf_status_string(s) != NULL && strlen(sf_status_string(s)) > 0);
  EXPECT(sf_version() > 0);

  // sf_gemm argument validation (before any HIP call)
  EXPECT(sf_gemm(0, 1, -1, 4, 4, 1, P(256), 4, 0, P(512), 4, 0, P(1024), 4, 0, SF_BF16, SF_BF16, 1.f, NULL,
                 SF_EPI_NONE, NULL) == SF_ERR_INVALID_ARG);
  EXPECT(strstr(sf_last_error(), "negative size") != NULL);
  EXPECT(sf_gemm(0, 1, 4, 4, 4, 1, P(256), 4, 0, P(512), 4, 0, P(1024), 4, 0, (sf_dtype)7, SF_BF16, 1.f, NULL,
                 SF_EPI_NONE, NULL) == SF_ERR_INVALID_ARG);
  EXPECT(sf_gemm(0, 1, 4, 4, 4, 1, P(256), 4, 0, P(512), 4, 0, P(1024), 4, 0, SF_BF16, SF_BF16, 1.f, NULL,
                 (sf_epilogue)9, NULL) == SF_ERR_INVALID_ARG);
  EXPECT(sf_gemm(0, 1, 4, 4, 4, 1, P(256), 4, 0, P(512), 4, 0, P(1024), 4, 0, SF_BF16, SF_BF16, 1.f, NULL,
                 SF_EPI_BIAS, NULL) == SF_ERR_INVALID_ARG);
  EXPECT(sf_gemm(0, 1, 4, 4, 4, 1, P(256), 3, 0, P(512), 4, 0, P(1024), 4, 0, SF_BF16, SF_BF16, 1.f, NULL,
                 SF_EPI_NONE, NULL) == SF_ERR_INVALID_ARG);
  EXPECT(sf_gemm(0, 1, 4, 4, 4, 3, P(256), 4, 16, P(512), 4, 16, P(1024), 4, 2, SF_BF16, SF_BF16, 1.f, NULL,
                 SF_EPI_NONE, NULL) == SF_ERR_INVALID_ARG);  // overlapping batch entries of C
  EXPECT(sf_gemm(0, 1, (int64_t)1 << 40, 4, 4, 1, P(256), 4, 0, P(512), 4, 0, P(1024), 4, 0, SF_BF16, SF_BF16,
                 1.f, NULL, SF_EPI_NONE, NULL) == SF_ERR_INVALID_ARG);
  EXPECT(sf_gemm(0, 1, 0, 4, 4, 1, NULL, 4, 0, NULL, 4, 0, NULL, 4, 0, SF_BF16, SF_BF16, 1.f, NULL, SF_EPI_NONE,
                 NULL) == SF_OK);  // empty problem: no-op
  EXPECT(sf_gemm_add(0, 1, 4, 4, 4, 1, P(256), 4, 0, P(512), 4, 0, P(1024), 4, 0, SF_BF16, SF_BF16, 1.f, NULL,
                     SF_EPI_NONE, NULL, 4, 0, NULL) == SF_ERR_INVALID_ARG);

  // The planner over a grid of shapes, dtypes, layouts and epilogues: every
  // plan text is a bounded, NUL-terminated string.
  const int64_t dims[] = {1, 2, 15, 16, 17, 63, 64, 65, 100, 127, 128, 129, 255, 256, 1000, 1920, 4096, 7680, 11008,
                          17776};
  const sf_dtype dts[] = {SF_F32, SF_F16, SF_BF16};
  char buf[96];
  long plans = 0;
  for (int ta = 0; ta < 2; ++ta)
    for (int tb = 0; tb < 2; ++tb)
      for (sf_dtype dt : dts)
        for (int64_t m : dims)
          for (int64_t n : dims)
            for (int64_t k : {(int64_t)64, (int64_t)128, (int64_t)1920, (int64_t)4096, (int64_t)4000}) {
              const int64_t lda = ta ? m : k, ldb = tb ? k : n;
              for (int64_t batch : {(int64_t)1, (int64_t)3}) {
                const int64_t sa = batch > 1 ? (ta ? k * m : m * k) : 0, sb = batch > 1 ? k * n : 0;
                const int64_t sc = batch > 1 ? m * n : 0;
                memset(buf, 'x', sizeof buf);
                const int rc = sf_gemm_plan(ta, tb, m, n, k, batch, P(256), lda, sa, P(4096), ldb, sb, P(65536), n,
                                            sc, dt, dt, 1.f, NULL, SF_EPI_NONE, buf, (int)sizeof buf);
                EXPECT(rc == SF_OK);
                EXPECT(memchr(buf, 0, sizeof buf) != NULL);
                ++plans;
              }
            }
  EXPECT(plans > 10000);
  // a plan for other CU counts (host-only override)
  setenv("SF_PLAN_CU_COUNT", "1024", 1);
  EXPECT(sf_gemm_noalloc(1, 0, 2816, 2816, 4096, 1, P(256), 2816, 0, P(512), 2816, 0, P(1024), 2816, 0, SF_BF16,
                         SF_BF16, 1.f, NULL, SF_EPI_NONE, NULL) == SF_ERR_UNSUPPORTED);
  EXPECT(strstr(sf_last_error(), "scratch") != NULL);
  for (const char* cus : {"248", "250", "7", "3"}) {
    setenv("SF_PLAN_CU_COUNT", cus, 1);
    EXPECT(sf_gemm_plan(0, 1, 17776, 1920, 7680, 1, P(256), 7680, 0, P(512), 7680, 0, P(1024), 1920, 0, SF_BF16,
                        SF_BF16, 1.f, NULL, SF_EPI_NONE, buf, (int)sizeof buf) == SF_OK);
  }
  unsetenv("SF_PLAN_CU_COUNT");

  // other entry points' validation
  // head sizes: multiples of 8 up to 64 run fused; others are refused
  EXPECT(sf_attention(P(256), 80, 0, P(256), 80, 0, P(256), 80, 0, P(256), 80, 0, 1, 64, 64, 72, 1.f, SF_F16, NULL) ==
         SF_ERR_UNSUPPORTED);
  EXPECT(sf_attention(P(256), 64, 0, P(256), 64, 0, P(256), 64, 0, P(256), 64, 0, 1, 64, 64, 36, 1.f, SF_F16, NULL) ==
         SF_ERR_UNSUPPORTED);
  EXPECT(sf_attention(P(256), 64, 0, P(256), 64, 0, P(256), 64, 0, P(256), 64, 0, 1, 64, 0, 64, 1.f, SF_F16, NULL) ==
         SF_ERR_INVALID_ARG);
  EXPECT(sf_layer_norm(P(256), P(256), 4, 0, NULL, NULL, 1e-5f, NULL, NULL, 0, 0, NULL, NULL, SF_BF16, NULL) ==
         SF_ERR_INVALID_ARG);
  EXPECT(sf_rms_norm(NULL, P(256), 4, 4, NULL, 1e-5f, SF_BF16, NULL) == SF_ERR_INVALID_ARG);
  EXPECT(sf_softmax_rows(P(256), P(256), -1, 4, SF_F32, SF_F32, 1.f, NULL) == SF_ERR_INVALID_ARG);
  EXPECT(sf_sum_dim(P(256), P(256), 1, -3, 4, SF_F32, SF_F32, NULL) == SF_ERR_INVALID_ARG);
  EXPECT(sf_cast(P(256), (sf_dtype)5, P(256), SF_F32, 4, NULL) == SF_ERR_INVALID_ARG);

  // runtime wrappers without a device: failures reported, never a crash
  int count = -1;
  (void)sf_get_device_count(&count);
  void* ptr = NULL;
  size_t got = 0;
  EXPECT(sf_cache_alloc(0, 1024, &ptr, &got) != SF_OK && ptr == NULL);
  EXPECT(sf_cache_alloc(0, 1024, NULL, &got) == SF_ERR_INVALID_ARG);
  EXPECT(strlen(sf_last_error()) < 512);
  EXPECT(sf_gemm(0, 1, 64, 64, 64, 1, P(256), 64, 0, P(8448), 64, 0, P(16640), 64, 0, SF_BF16, SF_BF16, 1.f, NULL,
                 SF_EPI_NONE, NULL) != SF_OK);  // valid arguments, no device

  if (g_bad) {
    fprintf(stderr, "%d expectation(s) failed\n", g_bad);
    return 1;
  }
  printf("abi host check: %ld plans, all expectations hold\n", plans);
  return 0;
}
