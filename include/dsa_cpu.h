/*
 * dsa_cpu.h -- C ABI of the host k-th-largest library (libdsa_cpu.so) used by
 * the CPU-offload ("hybrid") DSA path: the indexer scores are copied to pinned
 * host memory, their per-row thresholds computed on the host cores, and the
 * thresholds copied back for the GPU sparse attention
 * (reference dsa_hybrid.py:36-66).
 *
 * Built with g++ (OpenMP), no GPU code.  Every entry point validates its
 * arguments first, returns DSA_CPU_OK (0) or a negative code, and records a
 * message for a non-zero return, read back with dsa_cpu_last_error() on the
 * same thread.
 */
#ifndef DSA_CPU_H
#define DSA_CPU_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum dsa_cpu_status {
  DSA_CPU_OK = 0,
  DSA_CPU_EINVAL = -1, /* bad size, null pointer, k out of range, ... */
  DSA_CPU_ENOMEM = -3  /* a per-thread candidate buffer could not be allocated */
};

enum dsa_cpu_isa { DSA_CPU_ISA_SCALAR = 0, DSA_CPU_ISA_AVX512 = 1 };

/* Thread-local text of the last non-zero return on this thread. */
const char* dsa_cpu_last_error(void);

/* Instruction set the row scan uses on this host: AVX-512F when present,
 * unless the environment sets DSA_CPU_ISA=scalar (read on first use). */
int dsa_cpu_isa(void);

/*
 * k-th largest of every row of a host fp32 matrix, ties counted:
 *   thr[r] = torch.topk(row r, k).values[-1]        (NaN ranks above +inf)
 *
 *   scores    host pointer, `rows` rows of `n` values, row r at scores + r*ld
 *   k         1 <= k <= n
 *   causal_T  0: full rows.  > 0: rows are query rows of [.., causal_T,
 *             causal_T] causal indexer scores (n >= causal_T): row r is query
 *             t = (row0 + r) % causal_T and reads only its first t + 1
 *             entries, the others count as -inf, and rows with fewer than k
 *             read entries get -inf -- the full-row result when the indexer
 *             has written -inf above the diagonal.
 *   row0      causal mode: position of the first row in the flattened
 *             [.., causal_T] query rows (so a block of rows can start inside a
 *             batch element); >= 0, ignored for full rows.
 *   thr       host pointer, rows values
 *   nthreads  OpenMP threads; 0 = the OpenMP default (OMP_NUM_THREADS)
 *
 * Replaces: topk_threshold / topk_threshold_batch_merge of the reference's
 * AVX-512 extension (topk_avx512.cpp:226-264), whose output tensor
 * sizes[:-1] + [1] is exactly `thr` here; its TORCH_CHECKs (contiguous, fp32,
 * CPU, k > 0, k <= N; topk_avx512.cpp:227-234) are DSA_CPU_EINVAL.
 */
int dsa_cpu_topk_threshold(const float* scores, int64_t rows, int64_t n, int64_t ld, int k,
                           int64_t causal_T, int64_t row0, float* thr, int nthreads);

#ifdef __cplusplus
}
#endif

#endif /* DSA_CPU_H */
