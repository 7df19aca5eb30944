/* Sanitizer driver for the CPU oracle (oracle/graph_oracle.c), test infrastructure only:
 * tests/test_oracle_sanitizers.py compiles it together with the oracle under
 * -fsanitize=address,undefined and runs it.  Every oracle entry point runs on edge cases
 * (no atoms, one atom, a cell smaller than the radius, partial PBC with atoms far outside
 * the cell, a skewed cell, explicit targets with duplicates, both position dtypes); the
 * checks are invariants the definition fixes (degrees add up to the edge count, a full
 * graph is symmetric under (i, j, S) -> (j, i, -S), every edge is within the radius, the
 * filter at the same radius keeps everything), and the sanitizers catch any out-of-bounds
 * access or undefined behaviour on the way.  Exit status 0 on success. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

void* orc_graph_count(const void* pos, int f64, int64_t n, const double* cell, const uint8_t* pbc,
                      double radius, const int64_t* tgt, int64_t nt, int32_t* counts_user,
                      int64_t* total, int threads);
void orc_graph_write(void* hv, int64_t* src, int64_t* dst, int32_t* shift, double* vec, double* d2);
void orc_graph_free(void* hv);
int64_t orc_graph_num_images(void* hv);
void orc_edge_vectors(const void* pos, int f64, const double* cell, int64_t E, const int64_t* src,
                      const int64_t* dst, const int32_t* shift, double* vec, double* d2);
int64_t orc_filter_edges(const void* pos, int f64, const double* cell, double radius, int64_t E,
                         const int64_t* src, const int64_t* dst, const int32_t* shift, uint8_t* keep);
void orc_ref32_decide(const float* pos, int64_t n, const double* cell_d, const uint8_t* pbc,
                      double radius_d, int64_t E, const int64_t* src, const int64_t* dst,
                      const int32_t* shift, uint8_t* keep);
void orc_sfc_bounds(const float* pos, int64_t n, float* mn, float* range);
void orc_morton_keys(const float* pos, int64_t n, const float* mn, const float* range, int64_t* keys,
                     int threads);
void orc_hilbert_keys(const float* pos, int64_t n, const float* mn, const float* range, int64_t* keys);
void orc_sfc_labels(const int64_t* perm, int64_t n, int64_t W, const int64_t* weights, int64_t* labels);

static int failures = 0;
#define CHECK(c, ...)                                             \
    do {                                                          \
        if (!(c)) {                                               \
            fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__);  \
            fprintf(stderr, __VA_ARGS__);                         \
            fprintf(stderr, "\n");                                \
            failures++;                                           \
        }                                                         \
    } while (0)

static uint64_t rng_state = 88172645463325252ull;
static double urand(void)
{
    rng_state ^= rng_state << 13;
    rng_state ^= rng_state >> 7;
    rng_state ^= rng_state << 17;
    return (double)(rng_state >> 11) / 9007199254740992.0;
}

/* one case: build, check the invariants, run the neighbouring entry points on its edges */
static void run_case(const char* name, int64_t n, const double* cell, const uint8_t* pbc, double r,
                     double lo, double hi, int f64, const int64_t* tgt, int64_t nt)
{
    double* pd = (double*)malloc(sizeof(double) * 3 * (n ? n : 1));
    float* pf = (float*)malloc(sizeof(float) * 3 * (n ? n : 1));
    for (int64_t i = 0; i < n; i++) {
        double f[3] = {lo + (hi - lo) * urand(), lo + (hi - lo) * urand(), lo + (hi - lo) * urand()};
        for (int a = 0; a < 3; a++) {
            pd[3 * i + a] = f[0] * cell[a] + f[1] * cell[3 + a] + f[2] * cell[6 + a];
            pf[3 * i + a] = (float)pd[3 * i + a];
        }
    }
    if (!f64)
        for (int64_t i = 0; i < 3 * n; i++) pd[i] = pf[i];
    const void* pos = f64 ? (const void*)pd : (const void*)pf;
    const int64_t T = tgt ? nt : n;
    int32_t* counts = (int32_t*)malloc(sizeof(int32_t) * (T ? T : 1));
    int64_t E = -1;
    void* h = orc_graph_count(pos, f64, n, cell, pbc, r, tgt, nt, counts, &E, 1);
    CHECK(h != NULL, "%s: count failed", name);
    if (!h) { free(pd); free(pf); free(counts); return; }
    (void)orc_graph_num_images(h);
    int64_t sum = 0;
    for (int64_t t = 0; t < T; t++) sum += counts[t];
    CHECK(sum == E, "%s: degrees add up to %lld, edges %lld", name, (long long)sum, (long long)E);
    const int64_t Ea = E ? E : 1;
    int64_t* src = (int64_t*)malloc(sizeof(int64_t) * Ea);
    int64_t* dst = (int64_t*)malloc(sizeof(int64_t) * Ea);
    int32_t* sh = (int32_t*)malloc(sizeof(int32_t) * 3 * Ea);
    double* vec = (double*)malloc(sizeof(double) * 3 * Ea);
    double* d2 = (double*)malloc(sizeof(double) * Ea);
    orc_graph_write(h, src, dst, sh, vec, d2);
    orc_graph_free(h);
    for (int64_t e = 0; e < E; e++) {
        CHECK(src[e] >= 0 && src[e] < n && dst[e] >= 0 && dst[e] < n, "%s: edge %lld out of range", name,
              (long long)e);
        CHECK(d2[e] <= r * r && d2[e] > 1e-8, "%s: edge %lld at d2 %g", name, (long long)e, d2[e]);
    }
    if (!tgt) {  /* full graph: every (i, j, S) has its (j, i, -S) -- an O(E^2) check, small E */
        if (E <= 20000)
            for (int64_t e = 0; e < E; e++) {
                int found = 0;
                for (int64_t f = 0; f < E && !found; f++)
                    found = src[f] == dst[e] && dst[f] == src[e] && sh[3 * f] == -sh[3 * e] &&
                            sh[3 * f + 1] == -sh[3 * e + 1] && sh[3 * f + 2] == -sh[3 * e + 2];
                CHECK(found, "%s: edge %lld has no mirror", name, (long long)e);
            }
    }
    double* vec2 = (double*)malloc(sizeof(double) * 3 * Ea);
    double* d22 = (double*)malloc(sizeof(double) * Ea);
    orc_edge_vectors(pos, f64, cell, E, src, dst, sh, vec2, d22);
    CHECK(E == 0 || memcmp(d2, d22, sizeof(double) * E) == 0, "%s: edge_vectors differ", name);
    uint8_t* keep = (uint8_t*)malloc(Ea);
    CHECK(orc_filter_edges(pos, f64, cell, r, E, src, dst, sh, keep) == E, "%s: filter dropped edges", name);
    orc_ref32_decide(pf, n, cell, pbc, r, E, src, dst, sh, keep);
    if (n > 0) {
        float mn[3], range[3];
        int64_t* keys = (int64_t*)malloc(sizeof(int64_t) * n);
        int64_t* perm = (int64_t*)malloc(sizeof(int64_t) * n);
        int64_t* w = (int64_t*)malloc(sizeof(int64_t) * n);
        int64_t* lab = (int64_t*)malloc(sizeof(int64_t) * n);
        orc_sfc_bounds(pf, n, mn, range);
        orc_morton_keys(pf, n, mn, range, keys, 1);
        orc_hilbert_keys(pf, n, mn, range, keys);
        for (int64_t i = 0; i < n; i++) { perm[i] = n - 1 - i; w[i] = (i * 7) % 5; }
        for (int64_t W = 1; W <= 5; W += 2) {
            orc_sfc_labels(perm, n, W, NULL, lab);
            orc_sfc_labels(perm, n, W, w, lab);
            for (int64_t i = 0; i < n; i++) CHECK(lab[i] >= 0 && lab[i] < W, "%s: label out of range", name);
        }
        free(keys); free(perm); free(w); free(lab);
    }
    free(pd); free(pf); free(counts); free(src); free(dst); free(sh); free(vec); free(d2);
    free(vec2); free(d22); free(keep);
}

int main(void)
{
    const uint8_t all[3] = {1, 1, 1}, part[3] = {1, 0, 1}, none[3] = {0, 0, 0};
    const double cube[9] = {12, 0, 0, 0, 12, 0, 0, 0, 12};
    const double small[9] = {3, 0, 0, 0, 3.5, 0, 0, 0, 4};
    const double skew[9] = {14, 0, 0, 3.5, 13, 0, -2.5, 4, 12};
    const double general[9] = {11, 1.5, -0.7, 2.2, 12, 1.1, -1.4, 0.9, 10};
    int64_t tg[40];
    for (int i = 0; i < 40; i++) tg[i] = (i * 13) % 60;
    run_case("empty", 0, cube, all, 4.0, 0, 1, 0, NULL, 0);
    run_case("one atom", 1, cube, all, 4.0, 0, 1, 1, NULL, 0);
    run_case("one atom, cell smaller than r", 1, small, all, 7.5, 0, 1, 0, NULL, 0);
    run_case("cube", 300, cube, all, 3.5, 0, 1, 0, NULL, 0);
    run_case("cube fp64", 300, cube, all, 3.5, 0, 1, 1, NULL, 0);
    run_case("partial pbc, far outside", 120, cube, part, 4.0, -2.5, 3.5, 0, NULL, 0);
    run_case("no pbc", 150, cube, none, 4.0, -0.5, 1.5, 1, NULL, 0);
    run_case("small cell, many images", 12, small, all, 8.0, -1, 2, 1, NULL, 0);
    run_case("skewed", 200, skew, all, 4.5, 0, 1, 0, NULL, 0);
    run_case("general", 200, general, part, 4.5, -1, 2, 1, NULL, 0);
    run_case("targets with duplicates", 60, cube, all, 5.0, 0, 1, 0, tg, 40);
    if (failures) {
        fprintf(stderr, "%d failures\n", failures);
        return 1;
    }
    printf("oracle sanitizer driver: all cases passed\n");
    return 0;
}
