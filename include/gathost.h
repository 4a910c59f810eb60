/*
 * gathost.h -- host-side inputs for the GAT forward: seeded synthetic graphs
 * (destination-row CSR with one self-loop per node), node features and
 * weights.  Deterministic for a given seed, independent of the thread count.
 *
 * Replaces the reference's input makers: random_model
 * (baseline/src/common.cpp:50-62), the smoke fixture writer
 * (implementation/tools/prepare_smoke.py) and the converted OGB graphs
 * (implementation/tools/prepare_arxiv.py:18-50), which need raw data that is
 * not available offline; the synthetic graphs stand in for them at the same
 * N, E and degree skew.
 */
#ifndef GATHOST_H
#define GATHOST_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Row pointers of a uniform graph: row i has 1 self-loop + extra_i distinct
 * random sources, extra_i uniform in [0, 2*(mean_degree-1)].  row has n+1
 * entries; returns E (row[n]). */
uint64_t gathost_uniform_rows(uint64_t n, uint32_t mean_degree, uint64_t seed, uint64_t* row);

/* Row pointers of a power-law graph with exactly `edges` CSR entries
 * (self-loops included) whose largest in-degree is max_degree: the extra
 * in-degree of the node of rank r (a seeded random ranking) is proportional
 * to (r+1)^-alpha, alpha solved so that rank 0 gets max_degree-1, rounded by
 * largest remainders.  Returns E (== edges) or 0 if the request is infeasible. */
uint64_t gathost_powerlaw_rows(uint64_t n, uint64_t edges, uint32_t max_degree, uint64_t seed,
                               uint64_t* row);

/* Fills col for rows made by the two functions above: per row the self-loop
 * and distinct uniform random sources != i, ascending. */
void gathost_fill_sources(uint64_t n, const uint64_t* row, uint64_t seed, uint32_t* col);

/* R-MAT graph (probabilities a, b, c, d = 1-a-b-c) on 2^scale nodes: `edges`
 * directed edges drawn, self-loops added, duplicates removed, destination-row
 * CSR with ascending sources.  Two calls: col == NULL returns E and fills row;
 * then col (E entries) is filled by a second call with the same arguments. */
uint64_t gathost_rmat(int scale, uint64_t edges, double a, double b, double c, uint64_t seed,
                      uint64_t* row, uint32_t* col);

/* count values ~ N(0,1) (Box-Muller on a counter-based generator). */
void gathost_normal(uint64_t count, uint64_t seed, float* out);

/* Glorot-uniform layer: W ~ U(+-sqrt(6/(in+heads*dim))) [in][heads*dim],
 * aL, aR ~ U(+-sqrt(6/(heads+dim))) [heads*dim]. */
void gathost_glorot_param(int in, int heads, int dim, uint64_t seed, float* w, float* al, float* ar);

/* random_model layer (baseline/src/common.cpp:50-62): mt19937(rng_seed),
 * normal_distribution<float>; W/sqrt(in), aL and aR /sqrt(dim). */
void gathost_random_param(int in, int heads, int dim, int rng_seed, float* w, float* al, float* ar);

#ifdef __cplusplus
}
#endif
#endif /* GATHOST_H */
