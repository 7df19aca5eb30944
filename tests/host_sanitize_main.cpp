// Host-side sanitizer driver for the library's C ABI, test infrastructure only:
// tests/test_host_sanitizers.py compiles the library's sources with AddressSanitizer and
// UndefinedBehaviorSanitizer on the host code (-fno-gpu-sanitize) together with this file
// and runs it without a GPU.  Only host entry points are called: the workspace sizes (the
// plan: cell geometry, grid, tiles, workspace layout, descriptor validation) on random
// and extreme descriptors -- NaN / infinite / singular / nearly flat / huge / skewed
// cells, radii from 1e-6 to 1e6 cell widths, atom and target counts up to 2^31 - 1 -- and
// the error text.  Checks: every call returns either a size or 0 with an error message,
// and a valid descriptor's size does not shrink when atoms are added.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <random>

#include "dynamis_graph.h"

static int failures = 0;
#define CHECK(c, ...)                                            \
    do {                                                         \
        if (!(c)) {                                              \
            fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
            fprintf(stderr, __VA_ARGS__);                        \
            fprintf(stderr, "\n");                               \
            failures++;                                          \
        }                                                        \
    } while (0)

static size_t size_of(const dg_graph_desc& d)
{
    const size_t s = dg_graph_workspace_size(&d);
    if (s == 0) CHECK(strlen(dg_last_error()) > 0, "size 0 without an error message");
    return s;
}

int main()
{
    std::mt19937_64 g(7);
    std::uniform_real_distribution<double> U(0.0, 1.0);
    const double specials[] = {0.0, -0.0, 1e-300, 1e-12, 1e-6, 1.0, 1e6, 1e12, 1e300,
                               INFINITY, -INFINITY, NAN};
    long valid = 0, refused = 0;
    for (int it = 0; it < 20000; ++it) {
        dg_graph_desc d;
        memset(&d, 0, sizeof d);
        const int kind = it % 8;
        const double L = pow(10.0, -3.0 + 9.0 * U(g));
        for (int k = 0; k < 9; ++k) d.cell[k] = (k % 4 == 0 ? L : 0.0);
        if (kind == 1)
            for (int k = 0; k < 9; ++k) d.cell[k] += (U(g) - 0.5) * L;
        if (kind == 2) d.cell[8] = L * pow(10.0, -12.0 * U(g));  // nearly flat
        if (kind == 3) d.cell[g() % 9] = specials[g() % 12];
        if (kind == 4) {  // singular: two equal rows
            for (int k = 0; k < 3; ++k) d.cell[3 + k] = d.cell[k];
        }
        if (kind == 5) d.cell[3] = 50.0 * L, d.cell[6] = -40.0 * L;  // very skewed
        const double rr = L * pow(10.0, -6.0 + 12.0 * U(g));
        d.radius = kind == 6 ? specials[g() % 12] : rr;
        const int64_t ns[] = {0, 1, 2, 7, 1000, 1 << 20, (int64_t)1 << 27, 0x7fffffffLL - 1, 0x7fffffffLL,
                              (int64_t)1 << 40, -1};
        d.n_atoms = ns[g() % 11];
        d.has_targets = (int32_t)(g() % 2);
        d.n_targets = ns[g() % 11];
        d.pos_dtype = (int32_t)(g() % 3);  // 2: not a position dtype
        for (int k = 0; k < 3; ++k) d.pbc[k] = (uint8_t)(g() % 2);
        const size_t s = size_of(d);
        if (s) {
            ++valid;
            CHECK(d.n_atoms >= 0 && d.n_atoms <= 0x7fffffffLL, "accepted n_atoms %lld", (long long)d.n_atoms);
            CHECK(isfinite(d.radius) && d.radius > 0, "accepted radius %g", d.radius);
            if (d.n_atoms < 1000000 && d.n_atoms > 0) {  // more atoms never need less workspace
                dg_graph_desc e = d;
                e.n_atoms = d.n_atoms * 2;
                if (!d.has_targets) {
                    const size_t s2 = size_of(e);
                    CHECK(s2 == 0 || s2 >= s, "workspace shrank %zu -> %zu", s, s2);
                }
            }
        } else {
            ++refused;
        }
        // the other host entries
        (void)dg_filter_workspace_size(d.n_atoms);
        (void)dg_sfc_workspace_size(d.n_atoms);
        (void)dg_halo_workspace_size(d.n_atoms, (int64_t)(g() % 70) - 3);
        dg_batch_desc b;
        memset(&b, 0, sizeof b);
        b.n_images = ns[g() % 11];
        b.n_atoms = ns[g() % 11];
        b.pos_dtype = d.pos_dtype;
        b.radius = d.radius;
        (void)dg_batch_workspace_size(&b);
    }
    printf("host sanitizer driver: %ld descriptors accepted, %ld refused\n", valid, refused);
    if (failures) {
        fprintf(stderr, "%d failures\n", failures);
        return 1;
    }
    printf("all checks passed\n");
    return 0;
}
