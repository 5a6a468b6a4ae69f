// C-ABI shim over the reference's own CPU path, so Python tests and bench.py
// can call it. TEST INFRASTRUCTURE ONLY. It is compiled together with the
// reference's unmodified src/ops.cpp and src/threadpool.cpp (read in place from
// the reference checkout, never copied) by oracle/Makefile into
// oracle/_ref/libieref.so. Nothing here restates the reference: each function
// forwards to the reference function it names.
#include <cstdint>

#include "ops.h"         // reference: src/ops.h
#include "threadpool.h"  // reference: src/threadpool.h

extern "C" {

// ie::rope, src/ops.cpp:34-55
void ref_rope(float* x, int T, int n_heads, int head_dim, int pos0, float theta) {
  ie::rope(x, T, n_heads, head_dim, pos0, theta);
}

// ie::softmax, src/ops.cpp:57-66
void ref_softmax(float* x, int n) { ie::softmax(x, n); }

// ie::attention, src/ops.cpp:70-108 (runs on the reference's thread pool)
void ref_attention(float* out, const float* q, const float* k, const float* v, int T, int pos0,
                   int n_heads, int n_kv_heads, int head_dim) {
  ie::attention(out, q, k, v, T, pos0, n_heads, n_kv_heads, head_dim);
}

// ie::set_num_threads / thread_pool / physical_cores, src/threadpool.cpp:92-147
void ref_set_num_threads(int n) { ie::set_num_threads(n); }
int ref_num_threads() { return ie::thread_pool().num_threads(); }
int ref_physical_cores() { return ie::physical_cores(); }

}  // extern "C"
