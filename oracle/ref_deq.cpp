// Test infrastructure: re-exports the CPU dequantizer that the reference's
// own GPU test harness carries (gpu/test_matvec.cu:17-70), compiled from the
// file where it lies.  Used only to cross-check oracle/kq_oracle.c.
#define main aspida_reference_test_matvec_main
#include REF_SRC
#undef main

extern "C" void ref_deq_block(int kind, const uint8_t *blk, float *out) { deq_any(kind, blk, out); }
extern "C" int ref_block_bytes(int kind) { return bsz_of(kind); }
