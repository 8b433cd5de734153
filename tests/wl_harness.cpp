// CPU harness for the ragged work list's rules (mla-cuda_amd/csrc/worklist.h): built with
// g++ by tests/test_worklist_cpu.py and called through ctypes.  It exposes the very
// functions the device builder calls, so the test can drive them over adversarial inputs.
#include "worklist.h"

extern "C" {

int wl_harness_max_items(int B, int row_tiles) { return mla::wl_max_items(B, row_tiles); }

int wl_harness_ints(int B, int max_items) { return mla::wl_ints(B, max_items); }

int wl_harness_dense_keys(int Sk, int base, int block_keys) {
    return mla::dense_keys_per_split(Sk, base, block_keys);
}

int wl_harness_build(const int* seq_lens, int B, int Sk, int row_tiles, int block_keys,
                     int max_items, int* wl) {
    return mla::wl_build_serial(seq_lens, B, Sk, row_tiles, block_keys, max_items, wl);
}

int wl_harness_bucket(int L, int chunk) { return mla::wl_bucket(L, chunk); }

int wl_harness_thread_first(int tid, int B) { return mla::wl_thread_first(tid, B); }

}
