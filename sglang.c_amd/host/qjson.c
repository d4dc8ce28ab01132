/* qjson.c — a small recursive-descent JSON reader, enough for config.json's
 * quantization_config.  Objects keep key order; lookups return the first matching key. */
#include <stdlib.h>
#include <string.h>

#include "qhost.h"

typedef struct {
  const char *p, *end;
  int depth;
} qj_in;

static void ws(qj_in *s) {
  while (s->p < s->end && (*s->p == ' ' || *s->p == '\t' || *s->p == '\n' || *s->p == '\r'))
    s->p++;
}

static qj *mk(qj_type t) {
  qj *j = (qj *)calloc(1, sizeof(qj));
  if (j) j->type = t;
  return j;
}

static int push(qj *c, char *key, qj *v) {
  qj **ni = (qj **)realloc(c->items, sizeof(qj *) * (size_t)(c->count + 1));
  if (!ni) return 0;
  c->items = ni;
  if (c->type == QJ_OBJ) {
    char **nk = (char **)realloc(c->keys, sizeof(char *) * (size_t)(c->count + 1));
    if (!nk) return 0;
    c->keys = nk;
    c->keys[c->count] = key;
  }
  c->items[c->count++] = v;
  return 1;
}

static void utf8(char **o, unsigned cp) {
  char *q = *o;
  if (cp < 0x80) {
    *q++ = (char)cp;
  } else if (cp < 0x800) {
    *q++ = (char)(0xC0 | (cp >> 6));
    *q++ = (char)(0x80 | (cp & 0x3F));
  } else {
    *q++ = (char)(0xE0 | (cp >> 12));
    *q++ = (char)(0x80 | ((cp >> 6) & 0x3F));
    *q++ = (char)(0x80 | (cp & 0x3F));
  }
  *o = q;
}

static char *str(qj_in *s) {
  if (s->p >= s->end || *s->p != '"') return NULL;
  s->p++;
  const char *b = s->p;
  while (s->p < s->end && *s->p != '"') s->p += (*s->p == '\\') ? 2 : 1;
  if (s->p >= s->end) return NULL;
  char *out = (char *)malloc((size_t)(s->p - b) + 1), *o = out;
  if (!out) return NULL;
  for (const char *q = b; q < s->p; q++) {
    if (*q != '\\') {
      *o++ = *q;
      continue;
    }
    q++;
    switch (*q) {
      case 'n': *o++ = '\n'; break;
      case 't': *o++ = '\t'; break;
      case 'r': *o++ = '\r'; break;
      case 'b': *o++ = '\b'; break;
      case 'f': *o++ = '\f'; break;
      case 'u': {
        unsigned cp = 0;
        for (int i = 1; i <= 4 && q + i < s->p; i++) {
          const char c = q[i];
          cp = cp * 16 + (unsigned)(c >= '0' && c <= '9' ? c - '0' : (c | 32) - 'a' + 10);
        }
        q += 4;
        utf8(&o, cp);
        break;
      }
      default: *o++ = *q; break;
    }
  }
  *o = 0;
  s->p++;
  return out;
}

static qj *value(qj_in *s) {
  ws(s);
  if (s->p >= s->end || ++s->depth > 64) return NULL;
  qj *out = NULL;
  const char c = *s->p;
  if (c == '{' || c == '[') {
    const int obj = c == '{';
    out = mk(obj ? QJ_OBJ : QJ_ARR);
    s->p++;
    ws(s);
    if (s->p < s->end && *s->p == (obj ? '}' : ']')) {
      s->p++;
    } else {
      for (;;) {
        char *key = NULL;
        if (obj) {
          ws(s);
          key = str(s);
          ws(s);
          if (!key || s->p >= s->end || *s->p != ':') {
            free(key);
            qj_free(out);
            return NULL;
          }
          s->p++;
        }
        qj *v = value(s);
        if (!v || !push(out, key, v)) {
          free(key);
          qj_free(v);
          qj_free(out);
          return NULL;
        }
        ws(s);
        if (s->p < s->end && *s->p == ',') {
          s->p++;
          continue;
        }
        if (s->p < s->end && *s->p == (obj ? '}' : ']')) {
          s->p++;
          break;
        }
        qj_free(out);
        return NULL;
      }
    }
  } else if (c == '"') {
    char *t = str(s);
    if (!t) return NULL;
    out = mk(QJ_STR);
    out->str = t;
  } else if (s->end - s->p >= 4 && !strncmp(s->p, "true", 4)) {
    out = mk(QJ_BOOL);
    out->boolean = 1;
    s->p += 4;
  } else if (s->end - s->p >= 5 && !strncmp(s->p, "false", 5)) {
    out = mk(QJ_BOOL);
    s->p += 5;
  } else if (s->end - s->p >= 4 && !strncmp(s->p, "null", 4)) {
    out = mk(QJ_NULL);
    s->p += 4;
  } else {
    char buf[64];
    size_t n = 0;
    while (s->p + n < s->end && n < sizeof(buf) - 1 && strchr("+-0123456789.eE", s->p[n])) n++;
    memcpy(buf, s->p, n);
    buf[n] = 0;
    char *e = NULL;
    const double d = strtod(buf, &e);
    if (n == 0 || e == buf) return NULL;
    out = mk(QJ_NUM);
    out->num = d;
    s->p += e - buf;
  }
  s->depth--;
  return out;
}

qj *qj_parse(const char *text, size_t len) {
  qj_in s = {text, text + len, 0};
  qj *j = value(&s);
  if (!j) return NULL;
  ws(&s);
  if (s.p != s.end) {
    qj_free(j);
    return NULL;
  }
  return j;
}

void qj_free(qj *j) {
  if (!j) return;
  for (int i = 0; i < j->count; i++) {
    qj_free(j->items[i]);
    if (j->keys) free(j->keys[i]);
  }
  free(j->items);
  free(j->keys);
  free(j->str);
  free(j);
}

const qj *qj_get(const qj *o, const char *key) {
  if (!o || o->type != QJ_OBJ) return NULL;
  for (int i = 0; i < o->count; i++)
    if (!strcmp(o->keys[i], key)) return o->items[i];
  return NULL;
}

const char *qj_str(const qj *o, const char *key, const char *def) {
  const qj *v = qj_get(o, key);
  return v && v->type == QJ_STR ? v->str : def;
}

/* numbers round half away from zero; booleans count as 0/1 (matches the engine's reader) */
int qj_int(const qj *o, const char *key, int def) {
  const qj *v = qj_get(o, key);
  if (!v) return def;
  if (v->type == QJ_BOOL) return v->boolean ? 1 : 0;
  if (v->type != QJ_NUM) return def;
  return (int)(v->num >= 0 ? v->num + 0.5 : v->num - 0.5);
}

int qj_bool(const qj *o, const char *key, int def) {
  const qj *v = qj_get(o, key);
  if (!v) return def;
  if (v->type == QJ_BOOL) return v->boolean ? 1 : 0;
  if (v->type == QJ_NUM) return v->num != 0.0;
  return def;
}
