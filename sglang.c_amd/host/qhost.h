/* qhost.h — private declarations of the C11 host layer (not installed). */
#ifndef SGL_QHOST_H
#define SGL_QHOST_H

#include <stddef.h>
#include <stdint.h>

#include "sglq_shim.h"

#define QH_API __attribute__((visibility("default")))

void qh_info(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
#define QH_ERR(...) sglq_log_error(__VA_ARGS__)

/* minimal JSON reader (objects, arrays, strings, numbers, literals) */
typedef enum { QJ_NULL, QJ_BOOL, QJ_NUM, QJ_STR, QJ_ARR, QJ_OBJ } qj_type;
typedef struct qj qj;
struct qj {
  qj_type type;
  double num;
  int boolean;
  char *str;
  qj **items;
  char **keys;
  int count;
};
qj *qj_parse(const char *text, size_t len);
void qj_free(qj *j);
const qj *qj_get(const qj *obj, const char *key);
const char *qj_str(const qj *obj, const char *key, const char *def);
int qj_int(const qj *obj, const char *key, int def);
int qj_bool(const qj *obj, const char *key, int def);

/* group planning: fills plan->{ngroups,gp,nsteps,kmap,kinv}; caller frees kmap and kinv */
int qh_plan_groups(sglq_plan *p, int64_t ngroups, const int32_t *gidx, int spc,
                   int32_t **kmap, int32_t **kinv);

/* W8 weight (sgl_matmul_w8a16 operands) into the device layout; NULL after logging on error */
sglq_dev *qh_build_w8(const int8_t *W, const float *sw, int64_t N, int64_t K, int dev);

#endif
