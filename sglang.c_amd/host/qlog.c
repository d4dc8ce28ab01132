/* qlog.c — one-line error/info logging of the host layer (stderr).  SGL_QLINEAR_LOG=0
 * silences info lines; errors are always printed, like the reference's SGL_ERROR. */
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

#include "qhost.h"

void sglq_log_error(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  fputs("[sgl-qlinear] ERROR ", stderr);
  vfprintf(stderr, fmt, ap);
  fputc('\n', stderr);
  va_end(ap);
}

void qh_info(const char *fmt, ...) {
  const char *e = getenv("SGL_QLINEAR_LOG");
  if (!e || atoi(e) < 2) return;
  va_list ap;
  va_start(ap, fmt);
  fputs("[sgl-qlinear] ", stderr);
  vfprintf(stderr, fmt, ap);
  fputc('\n', stderr);
  va_end(ap);
}
