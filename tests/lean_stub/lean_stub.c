/* Test stand-in runtime for lean/lean.h (see lean/lean.h in this directory): heap objects with
 * reference counts, scalar arrays, boxed scalars, strings and IO results, plus probes the tests call
 * through ctypes (stub_*). TEST INFRASTRUCTURE only. */
#include <lean/lean.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

enum { TAG_SARRAY = 248, TAG_STRING = 249, TAG_USIZE = 250, TAG_CTOR_OK = 0, TAG_CTOR_ERR = 1, TAG_USER_ERR = 7 };

typedef struct {
  lean_object hdr;
  lean_object* fields[2];
} ctor2;
typedef struct {
  lean_object hdr;
  size_t v;
} usize_obj;
typedef struct {
  lean_object hdr;
  char s[];
} string_obj;

static long g_live = 0;  /* heap objects alive */
static long g_freed_arrays = 0;

static int is_scalar(const lean_object* o) { return ((uintptr_t)o & 1) == 1; }

static lean_object* alloc_obj(size_t bytes, unsigned tag) {
  lean_object* o = (lean_object*)calloc(1, bytes);
  if (!o) {
    fprintf(stderr, "lean stub: out of memory\n");
    abort();
  }
  o->m_rc = 1;
  o->m_tag = tag;
  g_live++;
  return o;
}

lean_object* lean_alloc_sarray(unsigned elem_size, size_t size, size_t capacity) {
  lean_sarray_object* a = (lean_sarray_object*)alloc_obj(sizeof(lean_sarray_object) + elem_size * capacity + 8,
                                                         TAG_SARRAY);
  a->m_header.m_other = (unsigned)elem_size;
  a->m_size = size;
  a->m_capacity = capacity;
  return (lean_object*)a;
}
size_t lean_sarray_size(b_lean_obj_arg o) { return ((lean_sarray_object*)o)->m_size; }
double* lean_float_array_cptr(lean_object* o) { return (double*)((lean_sarray_object*)o)->m_data; }

void lean_inc(lean_object* o) {
  if (!is_scalar(o)) o->m_rc++;
}
void lean_dec(lean_object* o) {
  if (is_scalar(o)) return;
  if (o->m_rc <= 0) {
    fprintf(stderr, "lean stub: release of a dead object (tag %u)\n", o->m_tag);
    abort();
  }
  if (--o->m_rc > 0) return;
  if (o->m_tag == TAG_CTOR_OK || o->m_tag == TAG_CTOR_ERR || o->m_tag == TAG_USER_ERR) {
    ctor2* c = (ctor2*)o;
    if (c->fields[0]) lean_dec(c->fields[0]);
  }
  if (o->m_tag == TAG_SARRAY) g_freed_arrays++;
  g_live--;
  o->m_rc = -1;  /* poison: a later use aborts */
  free(o);
}

lean_object* lean_box(size_t n) { return (lean_object*)((n << 1) | 1); }
size_t lean_unbox(b_lean_obj_arg o) { return (size_t)o >> 1; }
lean_object* lean_box_usize(size_t n) {
  usize_obj* u = (usize_obj*)alloc_obj(sizeof(usize_obj), TAG_USIZE);
  u->v = n;
  return (lean_object*)u;
}
size_t lean_unbox_usize(b_lean_obj_arg o) { return ((usize_obj*)o)->v; }
lean_object* lean_mk_string(const char* s) {
  size_t n = strlen(s);
  string_obj* o = (string_obj*)alloc_obj(sizeof(string_obj) + n + 1, TAG_STRING);
  memcpy(o->s, s, n + 1);
  return (lean_object*)o;
}
static lean_object* ctor(unsigned tag, lean_object* a) {
  ctor2* c = (ctor2*)alloc_obj(sizeof(ctor2), tag);
  c->fields[0] = a;
  c->fields[1] = lean_box(0);  /* the world */
  return (lean_object*)c;
}
lean_object* lean_mk_io_user_error(lean_object* msg) { return ctor(TAG_USER_ERR, msg); }
lean_object* lean_io_result_mk_ok(lean_object* a) { return ctor(TAG_CTOR_OK, a); }
lean_object* lean_io_result_mk_error(lean_object* e) { return ctor(TAG_CTOR_ERR, e); }
void lean_internal_panic(const char* msg) {
  fprintf(stderr, "INTERNAL PANIC: %s\n", msg);
  fflush(stderr);
  abort();
}

/* ---- probes for the tests ---- */
LEAN_EXPORT lean_object* stub_array(const double* data, size_t n) {
  lean_object* a = lean_alloc_sarray(sizeof(double), n, n);
  if (n) memcpy(lean_float_array_cptr(a), data, 8 * n);
  return a;
}
LEAN_EXPORT size_t stub_array_size(lean_object* a) { return lean_sarray_size(a); }
LEAN_EXPORT const double* stub_array_data(lean_object* a) { return lean_float_array_cptr(a); }
LEAN_EXPORT int stub_rc(lean_object* o) { return is_scalar(o) ? 1 : o->m_rc; }
LEAN_EXPORT long stub_live(void) { return g_live; }
LEAN_EXPORT long stub_freed_arrays(void) { return g_freed_arrays; }
/* IO result: 1 ok, 0 error */
LEAN_EXPORT int stub_io_ok(lean_object* r) { return r->m_tag == TAG_CTOR_OK; }
LEAN_EXPORT lean_object* stub_io_value(lean_object* r) { return ((ctor2*)r)->fields[0]; }
LEAN_EXPORT const char* stub_io_error(lean_object* r) {
  lean_object* e = ((ctor2*)r)->fields[0];
  return ((string_obj*)((ctor2*)e)->fields[0])->s;
}
LEAN_EXPORT size_t stub_unbox(lean_object* o) { return is_scalar(o) ? lean_unbox(o) : lean_unbox_usize(o); }
LEAN_EXPORT void stub_release(lean_object* o) { lean_dec(o); }
