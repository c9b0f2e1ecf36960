// q8_tactics.h -- the shape-keyed matmul tactic table for gfx950.
//
// The reference keeps its kernel choices in a ranked table of tactics with
// guards, a maturity and a line of evidence (apps/engine/src/tactics.rs:118-181,
// 229-347), but its matmul regime switch is hard-coded (cuda/mod.rs:803-892).
// Here the matmul choice is such a table: each row guards a regime (n range)
// and derives its launch parameters from (n, out, k).
#ifndef Q8_TACTICS_H
#define Q8_TACTICS_H

#include "../../include/q8mi.h"

enum { Q8_MATURITY_REJECTED = 0, Q8_MATURITY_EXPERIMENTAL = 1, Q8_MATURITY_MEASURED = 2 };

struct Q8TacticRow {
    const char *name;
    int kernel;
    int n_min, n_max;
    int maturity;
    int rank;
    const char *evidence;
};

int q8_tactics_table_size();
const Q8TacticRow &q8_tactics_row(int i);
// Resolve the tactic for one matmul; cu_count sizes the grid heuristics.
int q8_tactics_choose(int n, int out, int k, int cu_count, q8_tactic *t);
// Launch shapes (slots = member tiles per GEMV workgroup: 2 for fused gate/up).
void q8_gemv_shape(int out, int k, int cu_count, int slots, q8_tactic *t);
void q8_gemm_shape(int n, int out, int k, int cu_count, q8_tactic *t);
void q8_gemm_h_shape(int n, int out, int k, int cu_count, q8_tactic *t);
/* Staged GEMM launch shape (RW, KW, TPW) for f16 (i8 = 0) or int8 (i8 = 1) activation units. */
void q8_gemm_staged_shape(int n, int out, int k, int cu_count, int i8, q8_tactic *t);
/* The prepared-activation format the table's choice for n consumes
 * (Q8_PREPARED_I8 or Q8_PREPARED_F16): it depends on n only. */
int q8_tactics_prepared_format(int n);
/* The first non-rejected row of `kernel` and its launch shape for (n, out, k). */
int q8_tactics_for_kernel(int kernel, int n, int out, int k, int cu_count, q8_tactic *t);

#endif
