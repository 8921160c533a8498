/*
 * pai_qgemm_shape_check against the reference executor's own GEMM/GEMV
 * branch (scheduler/scheduler.c:280-343, reached through pai_sched_execute
 * at scheduler.c:413-429), built from the reference's sources.
 *
 * Part 1, statuses: every combination of operand shapes drawn from ranks 1
 * and 2 with extents 1..3 (plus two rank-3 shapes), for GEMM and GEMV, runs
 * through a one-op graph in the reference executor; its status (OK or
 * MISMATCH) must equal pai_qgemm_shape_check's when the weight is given the
 * shape of the graph's weight operand, and the token count must be the
 * activation rows. An accepted case with a weight of another shape must be
 * rejected.
 *
 * Part 2, orientation: for the three accepted forms (GEMV, row vector,
 * GEMM) with a Q8_0 weight of unit scale and asymmetric integer codes, the
 * reference executor's result on the dequantized values laid out as its
 * graph expects (A = the weight rows for GEMV, B = the transposed weight
 * otherwise) equals the CPU twin pai_qgemm_ref_f32 bit for bit.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <graph/graph.h>
#include <scheduler/scheduler.h>

#include "pai_hip.h"

typedef struct {
  uint32_t rank;
  uint64_t d[3];
} shape_t;

static pai_graph_t g_graph;
static pai_sched_plan_t g_plan;

/* Build a one-op graph a, b -> c, run it, copy out c. a_data/b_data may
 * be NULL (zeros). */
static int ref_run(int is_gemv, const shape_t *a, const shape_t *b, const shape_t *c,
                   const float *a_data, const float *b_data, float *c_out) {
  pai_graph_mem_plan_t mp;
  pai_graph_init(&g_graph);
  pai_graph_value_id va = pai_graph_add_value(&g_graph, PAI_DTYPE_F32, a->rank, a->d, 0);
  pai_graph_value_id vb = pai_graph_add_value(&g_graph, PAI_DTYPE_F32, b->rank, b->d, 0);
  pai_graph_value_id vc = pai_graph_add_value(&g_graph, PAI_DTYPE_F32, c->rank, c->d, 0);
  if (va == 0 || vb == 0 || vc == 0) return 1000;
  pai_graph_value_id in[2] = {va, vb};
  pai_graph_value_id out[1] = {vc};
  if (pai_graph_add_op(&g_graph, is_gemv ? PAI_OP_GEMV : PAI_OP_GEMM, 2, 1, in, out) == 0)
    return 1001;
  pai_graph_set_input(&g_graph, va);
  pai_graph_set_input(&g_graph, vb);
  pai_graph_set_output(&g_graph, vc);
  if (pai_graph_memory_plan(&g_graph, &mp) != PAI_OK) return 1002;
  if (pai_sched_build(&g_graph, &mp, PAI_SCHED_INTERACTIVE, NULL, &g_plan) != PAI_OK) {
    pai_graph_mem_plan_free(&mp);
    return 1003;
  }
  uint8_t *region = (uint8_t *)calloc(1, (size_t)mp.region_bytes + 64);
  if (region == NULL) return 1004;
  if (a_data)
    memcpy(region + pai_graph_mem_plan_offset(&mp, va), a_data,
           g_graph.values[va].size_bytes);
  if (b_data)
    memcpy(region + pai_graph_mem_plan_offset(&mp, vb), b_data,
           g_graph.values[vb].size_bytes);
  int st = pai_sched_execute(&g_graph, &mp, &g_plan, region, NULL);
  if (st == PAI_OK && c_out)
    memcpy(c_out, region + pai_graph_mem_plan_offset(&mp, vc), g_graph.values[vc].size_bytes);
  free(region);
  pai_graph_mem_plan_free(&mp);
  return st;
}

static int shapes(shape_t *out) {
  int n = 0;
  for (uint64_t i = 1; i <= 3; i++) out[n++] = (shape_t){1, {i, 0, 0}};
  for (uint64_t i = 1; i <= 3; i++)
    for (uint64_t j = 1; j <= 3; j++) out[n++] = (shape_t){2, {i, j, 0}};
  out[n++] = (shape_t){3, {1, 1, 1}};
  out[n++] = (shape_t){3, {2, 3, 1}};
  return n;
}

static int part1(void) {
  shape_t s[16];
  const int ns = shapes(s);
  int runs = 0, accepted = 0, bad = 0;
  for (int gemv = 0; gemv <= 1; gemv++)
    for (int ia = 0; ia < ns; ia++)
      for (int ib = 0; ib < ns; ib++)
        for (int ic = 0; ic < ns; ic++) {
          const shape_t *a = &s[ia], *b = &s[ib], *c = &s[ic];
          const int want = ref_run(gemv, a, b, c, NULL, NULL, NULL);
          if (want != PAI_OK && want != PAI_ERR_MISMATCH) {
            printf("reference status %d\n", want);
            return 1;
          }
          /* the weight takes the shape of the graph's weight operand */
          uint64_t wn = 2, wk = 3;
          if (gemv && a->rank == 2) {
            wn = a->d[0];
            wk = a->d[1];
          } else if (!gemv && b->rank == 2) {
            wn = b->d[1];
            wk = b->d[0];
          }
          uint64_t m = 0;
          const int got = pai_qgemm_shape_check(gemv, a->rank, a->d, b->rank, b->d, c->rank,
                                                c->d, wn, wk, &m);
          runs++;
          if (got != want) {
            printf("status gemv=%d a=%u[%llu,%llu] b=%u[%llu,%llu] c=%u[%llu,%llu]: ref %d, "
                   "ours %d\n",
                   gemv, a->rank, (unsigned long long)a->d[0], (unsigned long long)a->d[1],
                   b->rank, (unsigned long long)b->d[0], (unsigned long long)b->d[1], c->rank,
                   (unsigned long long)c->d[0], (unsigned long long)c->d[1], want, got);
            bad++;
            continue;
          }
          if (want != PAI_OK) continue;
          accepted++;
          const uint64_t tokens = (gemv || a->rank == 1) ? 1u : a->d[0];
          if (m != tokens) {
            printf("tokens %llu, want %llu\n", (unsigned long long)m,
                   (unsigned long long)tokens);
            bad++;
          }
          uint64_t m2 = 0;
          if (pai_qgemm_shape_check(gemv, a->rank, a->d, b->rank, b->d, c->rank, c->d, wn + 1,
                                    wk, &m2) != PAI_ERR_MISMATCH ||
              pai_qgemm_shape_check(gemv, a->rank, a->d, b->rank, b->d, c->rank, c->d, wn,
                                    wk + 1, &m2) != PAI_ERR_MISMATCH) {
            printf("accepted a weight of another shape\n");
            bad++;
          }
        }
  printf("statuses: %d cases, %d accepted, %d differ\n", runs, accepted, bad);
  return bad != 0 || accepted == 0;
}

/* Q8_0 blocks of unit scale: 2-byte f16 scale, 32 signed codes. */
#define N_ROWS 3u
#define K_COLS 64u
#define ROW_BYTES (K_COLS / 32u * 34u)

static int part2(void) {
  uint8_t blocks[N_ROWS * ROW_BYTES];
  float wrow[N_ROWS * K_COLS]; /* [n][k], the dequantized rows */
  float wt[K_COLS * N_ROWS];   /* [k][n] */
  for (uint32_t r = 0; r < N_ROWS; r++)
    for (uint32_t b = 0; b < K_COLS / 32u; b++) {
      uint8_t *blk = blocks + r * ROW_BYTES + b * 34u;
      blk[0] = 0x00;
      blk[1] = 0x3C; /* f16 1.0 */
      for (uint32_t i = 0; i < 32u; i++) {
        const uint32_t col = b * 32u + i;
        const int code = (int)((r * 7u + col * 3u + col * col) % 11u) - 4;
        blk[2 + i] = (uint8_t)(int8_t)code;
        wrow[r * K_COLS + col] = (float)code;
        wt[col * N_ROWS + r] = (float)code;
      }
    }
  float x[2 * K_COLS];
  for (uint32_t i = 0; i < 2u * K_COLS; i++) x[i] = (float)((int)(i % 5u) - 2) * 0.5f;

  int bad = 0;
  float ref[2 * N_ROWS], twin[2 * N_ROWS];
  /* GEMV: A = the weight rows [n][k], b = x[k], c = y[n] */
  {
    const shape_t a = {2, {N_ROWS, K_COLS, 0}}, b = {1, {K_COLS, 0, 0}}, c = {1, {N_ROWS, 0, 0}};
    if (ref_run(1, &a, &b, &c, wrow, x, ref) != PAI_OK) return 1;
    if (pai_qgemm_ref_f32(8u, 1u, N_ROWS, K_COLS, x, blocks, twin) != PAI_OK) return 1;
    bad += memcmp(ref, twin, N_ROWS * sizeof(float)) != 0;
  }
  /* row vector: a = x[k], b = W^T [k][n], c = [1][n] */
  {
    const shape_t a = {1, {K_COLS, 0, 0}}, b = {2, {K_COLS, N_ROWS, 0}},
                  c = {2, {1, N_ROWS, 0}};
    if (ref_run(0, &a, &b, &c, x, wt, ref) != PAI_OK) return 1;
    if (pai_qgemm_ref_f32(8u, 1u, N_ROWS, K_COLS, x, blocks, twin) != PAI_OK) return 1;
    bad += memcmp(ref, twin, N_ROWS * sizeof(float)) != 0;
  }
  /* GEMM: a = X [2][k], b = W^T [k][n], c = [2][n] */
  {
    const shape_t a = {2, {2, K_COLS, 0}}, b = {2, {K_COLS, N_ROWS, 0}}, c = {2, {2, N_ROWS, 0}};
    if (ref_run(0, &a, &b, &c, x, wt, ref) != PAI_OK) return 1;
    if (pai_qgemm_ref_f32(8u, 2u, N_ROWS, K_COLS, x, blocks, twin) != PAI_OK) return 1;
    bad += memcmp(ref, twin, 2 * N_ROWS * sizeof(float)) != 0;
  }
  printf("orientation: %d of 3 forms differ\n", bad);
  return bad != 0;
}

int main(void) {
  if (part1() || part2()) return 1;
  printf("run_gemm parity ok\n");
  return 0;
}
