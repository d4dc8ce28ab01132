/* qload_fuzz.c — host-side sanitizer run over the safetensors reader and the quantized-weight
 * lookups (sgl_qst_*, sgl_qlinear_probe), built with -fsanitize=address,undefined by
 * tests/test_host_asan.py.  Header text is mutated at random; every result is allowed except
 * a sanitizer report.  The device-side create calls that sgl_qlinear_load would make are
 * stand-ins here: probe never reaches them. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "sgl/qload.h"
#include "sgl/qweight.h"
#ifndef ASAN_FUZZ_PATH
#define ASAN_FUZZ_PATH "qload_fuzz.st"
#endif
/* stand-ins for the device-side calls qload.c and qweight.c reach (never reached by probe) */
sgl_qlinear *sgl_qlinear_create(const sgl_qcfg *c, const int32_t *a, int64_t b, int64_t d, const int32_t *e, int64_t f, int64_t g, const float *h, int64_t i, int64_t j, const int32_t *k, int64_t l, int64_t m, int64_t n, int o) { return 0; }
sgl_qlinear *sgl_qlinear_create_marlin(const sgl_qcfg *c, const int32_t *a, int64_t b, int64_t d, const int32_t *e, int64_t f, int64_t g, const float *h, int64_t i, int64_t j, int64_t m, int64_t n, int o) { return 0; }
sgl_qlinear *sgl_qlinear_create_ct(const sgl_qcfg *c, const int32_t *a, int64_t b, int64_t d, const float *h, int64_t i, int64_t j, int64_t m, int64_t n, int o) { return 0; }
sgl_qlinear *sgl_qlinear_create_mxfp4(const uint8_t *a, int64_t b, int64_t d, const uint8_t *h, int64_t i, int64_t j, int64_t m, int64_t n, int o) { return 0; }
int sgl_q_pack(int bits) { return bits > 0 ? 32 / bits : 0; }
void sglq_log_error(const char *fmt, ...) { (void)fmt; }
void qh_info(const char *fmt, ...) { (void)fmt; }
static unsigned rs;
static unsigned rnd(void) { rs = rs * 1103515245u + 12345u; return rs >> 8; }
int main(int argc, char **argv) {
  rs = argc > 1 ? (unsigned)atoi(argv[1]) : 1u;
  const char *hdr = "{\"b.qweight\":{\"dtype\":\"I32\",\"shape\":[16,32],\"data_offsets\":[0,2048]},"
                    "\"b.qzeros\":{\"dtype\":\"I32\",\"shape\":[1,4],\"data_offsets\":[2048,2064]},"
                    "\"b.scales\":{\"dtype\":\"F16\",\"shape\":[1,32],\"data_offsets\":[2064,2128]}}";
  const size_t hl = strlen(hdr), dl = 2128;
  for (int it = 0; it < 20000; it++) {
    char buf[4096];
    size_t n = hl;
    memcpy(buf, hdr, hl);
    for (int k = 0, m = 1 + rnd() % 6; k < m; k++) {
      size_t i = n ? rnd() % n : 0;
      switch (rnd() % 3) {
        case 0: if (n) buf[i] = (char)rnd(); break;
        case 1: { size_t d = 1 + rnd() % 8; if (i + d > n) d = n - i; memmove(buf + i, buf + i + d, n - i - d); n -= d; } break;
        default: if (n + 4 < sizeof(buf)) { memmove(buf + i + 4, buf + i, n - i); for (int q = 0; q < 4; q++) buf[i + q] = "[{\":"[rnd() % 4]; n += 4; } break;
      }
    }
    FILE *f = fopen(ASAN_FUZZ_PATH, "wb");
    unsigned long long h64 = n;
    fwrite(&h64, 8, 1, f); fwrite(buf, 1, n, f);
    char *zeros = calloc(1, dl); fwrite(zeros, 1, dl, f); free(zeros); fclose(f);
    sgl_qst *st = sgl_qst_open(ASAN_FUZZ_PATH);
    if (!st) continue;
    for (int mth = 1; mth <= 4; mth++) {
      sgl_qcfg c; memset(&c, 0, sizeof(c));
      c.method = mth; c.bits = (rnd() & 1) ? 4 : 8; c.group_size = (rnd() & 1) ? 128 : -1;
      c.zero_point = rnd() & 1; c.layout = rnd() & 1;
      sgl_qload_info info;
      (void)sgl_qlinear_probe(&c, (sgl_qraw_fn)sgl_qst_get_raw, st, "b", &info);
    }
    sgl_qst_close(st);
    sgl_qcfg c2;
    (void)c2;
  }
  printf("asan fuzz done\n");
  return 0;
}
