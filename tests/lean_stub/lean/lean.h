/* Test stand-in for the parts of Lean 4's runtime header (lean/lean.h) that the pufferhip glue
 * uses: the object header, scalar arrays, boxing, strings, IO results and panics. TEST
 * INFRASTRUCTURE: it lets the tests compile the glue and call it through its Lean ABI without a Lean
 * toolchain. The object and scalar-array layouts follow Lean's (header word, then size, capacity and
 * the data); the functions live in lean_stub.c, which also counts releases so tests can check that
 * every owned argument is consumed. */
#ifndef PUFFERHIP_TEST_LEAN_STUB_H
#define PUFFERHIP_TEST_LEAN_STUB_H
#include <stddef.h>
#include <stdint.h>

#define LEAN_EXPORT __attribute__((visibility("default")))

typedef struct {
  int m_rc;
  unsigned m_cs_sz : 16;
  unsigned m_other : 8;
  unsigned m_tag : 8;
} lean_object;

typedef lean_object* lean_obj_arg;   /* owned argument */
typedef lean_object* b_lean_obj_arg; /* borrowed argument */
typedef lean_object* lean_obj_res;   /* owned result */

typedef struct {
  lean_object m_header;
  size_t m_size;
  size_t m_capacity;
  uint8_t m_data[];
} lean_sarray_object;

lean_object* lean_alloc_sarray(unsigned elem_size, size_t size, size_t capacity);
size_t lean_sarray_size(b_lean_obj_arg o);
double* lean_float_array_cptr(lean_object* o);
void lean_dec(lean_object* o);
void lean_inc(lean_object* o);
lean_object* lean_box(size_t n);
size_t lean_unbox(b_lean_obj_arg o);
lean_object* lean_box_usize(size_t n);
size_t lean_unbox_usize(b_lean_obj_arg o);
lean_object* lean_mk_string(const char* s);
lean_object* lean_mk_io_user_error(lean_object* msg);
lean_object* lean_io_result_mk_ok(lean_object* a);
lean_object* lean_io_result_mk_error(lean_object* e);
void lean_internal_panic(const char* msg);

#endif
