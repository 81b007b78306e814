/*
 * TEST INFRASTRUCTURE ONLY — the CPU oracle for the SOAP hot path.
 *
 * A plain-C restatement of the reference's neighbour graph and GTO SOAP
 * (nicheal/MDescriptor, C++17/OpenMP).  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load this library, and only as the
 * checker or the timed CPU baseline.  The product path (mdescriptor_amd)
 * never links, imports or calls it.
 *
 * Each function names the reference file:line it follows.  Parity status of
 * every function is pinned by tests (see tests/test_oracle_*.py):
 *   graph        : brute-force closed form over shifts, the reference's
 *                  NeighborList golden (448 pairs), boundary KATs, and the
 *                  reference C++ compiled in place (oracle/_ref)
 *   harmonics    : scipy sph_harm x r^l, orthonormality on a quadrature grid
 *   soap         : the reference's SOAP goldens (project + DScribe sidecar),
 *                  single-atom closed form, and oracle/_ref
 *   neighbor list: the reference's NeighborList goldens, the half/full
 *                  identity (full = half + its reversal, self pairs apart),
 *                  and oracle/_ref over every (full, self_pairs) setting
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define MDXO_PI 3.141592653589793238462643383279502884
#define MDXO_SQRT2 1.414213562373095048801688724209698079

/* status codes mirror the C-ABI of the product library */
enum { MDXO_OK = 0, MDXO_INVALID = 1, MDXO_NOMEM = 2, MDXO_CANCELLED = 4 };

static void set_error(char* err, int errlen, const char* message) {
    if (err != NULL && errlen > 0) {
        snprintf(err, (size_t)errlen, "%s", message);
    }
}

/* ------------------------------------------------------------------------ */
/* 3x3 helpers: cpp/include/mdescriptor/detail/math3.hpp:46-68              */
/* ------------------------------------------------------------------------ */
static double det3(const double* m) {
    return m[0] * (m[4] * m[8] - m[5] * m[7])
        - m[1] * (m[3] * m[8] - m[5] * m[6])
        + m[2] * (m[3] * m[7] - m[4] * m[6]);
}

static int inverse3(const double* m, double* r) {
    const double d = det3(m);
    if (!isfinite(d) || fabs(d) < 1e-14) return 0;
    r[0] = (m[4] * m[8] - m[5] * m[7]) / d;
    r[1] = (m[2] * m[7] - m[1] * m[8]) / d;
    r[2] = (m[1] * m[5] - m[2] * m[4]) / d;
    r[3] = (m[5] * m[6] - m[3] * m[8]) / d;
    r[4] = (m[0] * m[8] - m[2] * m[6]) / d;
    r[5] = (m[2] * m[3] - m[0] * m[5]) / d;
    r[6] = (m[3] * m[7] - m[4] * m[6]) / d;
    r[7] = (m[1] * m[6] - m[0] * m[7]) / d;
    r[8] = (m[0] * m[4] - m[1] * m[3]) / d;
    return 1;
}

/* batch validation: cpp/include/mdescriptor/detail/batch.hpp:19-80 */
static int validate_batch(const int32_t* numbers, const double* positions, const double* cells,
                          const int32_t* pbc, const int64_t* offsets, int64_t structures,
                          int64_t atoms, char* err, int errlen) {
    if (structures < 0 || atoms < 0 || offsets == NULL) {
        set_error(err, errlen, "invalid structure batch");
        return 0;
    }
    if (structures == 0) {
        if (atoms != 0 || offsets[0] != 0) {
            set_error(err, errlen, "empty structure batch has non-empty atom data");
            return 0;
        }
        return 1;
    }
    if (offsets[0] != 0 || offsets[structures] != atoms) {
        set_error(err, errlen, "offsets do not describe the flattened arrays");
        return 0;
    }
    for (int64_t s = 0; s < structures; ++s) {
        if (offsets[s] < 0 || offsets[s] > offsets[s + 1] || offsets[s + 1] > atoms) {
            set_error(err, errlen, "offsets must be monotonic");
            return 0;
        }
        int periodic = 1, isolated = 1;
        for (int a = 0; a < 3; ++a) {
            const int32_t f = pbc[s * 3 + a];
            if (f != 0 && f != 1) {
                set_error(err, errlen, "pbc must contain only 0 or 1");
                return 0;
            }
            periodic = periodic && f == 1;
            isolated = isolated && f == 0;
        }
        if (!periodic && !isolated) {
            set_error(err, errlen, "mixed periodicity is not supported; use all-zero or all-one pbc");
            return 0;
        }
        const double* cell = cells + s * 9;
        for (int i = 0; i < 9; ++i) {
            if (!isfinite(cell[i])) {
                set_error(err, errlen, "cells must be finite");
                return 0;
            }
        }
        const double d = det3(cell);
        if (periodic && (!isfinite(d) || fabs(d) < 1e-14)) {
            set_error(err, errlen, "cells must be nonsingular");
            return 0;
        }
    }
    for (int64_t i = 0; i < atoms; ++i) {
        if (numbers[i] <= 0) {
            set_error(err, errlen, "atomic numbers must be positive");
            return 0;
        }
        for (int a = 0; a < 3; ++a) {
            if (!isfinite(positions[i * 3 + a])) {
                set_error(err, errlen, "positions must be finite");
                return 0;
            }
        }
    }
    return 1;
}

/* ------------------------------------------------------------------------ */
/* Neighbour graph: cpp/src/common/neighbor.cpp:423-679 (image-extended     */
/* path, store_shifts = true, use_scaled_periodic_images = false)           */
/* ------------------------------------------------------------------------ */
typedef struct {
    int32_t atom;
    int32_t shift[3];
    double pos[3];
} ext_atom;

typedef struct {
    double minimum[3];
    double spacing[3];
    int dims[3];
    int64_t* offsets; /* cell_count + 1 */
    int32_t* atoms;   /* extended indices, cell-major, extended order within a cell */
} cell_grid;

/* CellGrid::coordinate, neighbor.cpp:122-132 */
static int grid_coordinate(const cell_grid* g, double value, int axis) {
    const double scaled = (value - g->minimum[axis]) / g->spacing[axis];
    if (!(scaled > 0.0)) return 0;
    if (!isfinite(scaled) || scaled >= (double)g->dims[axis]) return g->dims[axis] - 1;
    return (int)scaled;
}

static int64_t grid_index(const cell_grid* g, int x, int y, int z) {
    return (int64_t)x + (int64_t)g->dims[0] * ((int64_t)y + (int64_t)g->dims[1] * (int64_t)z);
}

/* build_grid, neighbor.cpp:135-194 */
static int build_grid(const ext_atom* ext, int64_t n_ext, double cutoff, cell_grid* g,
                      char* err, int errlen) {
    memset(g, 0, sizeof(*g));
    g->dims[0] = g->dims[1] = g->dims[2] = 1;
    if (n_ext == 0) {
        g->offsets = (int64_t*)calloc(2, sizeof(int64_t));
        return g->offsets != NULL;
    }
    double mn[3], mx[3];
    for (int a = 0; a < 3; ++a) mn[a] = mx[a] = ext[0].pos[a];
    for (int64_t i = 0; i < n_ext; ++i) {
        for (int a = 0; a < 3; ++a) {
            if (ext[i].pos[a] < mn[a]) mn[a] = ext[i].pos[a];
            if (ext[i].pos[a] > mx[a]) mx[a] = ext[i].pos[a];
        }
    }
    const double padding = 1e-10;
    for (int a = 0; a < 3; ++a) {
        mn[a] -= padding;
        mx[a] += padding;
        g->minimum[a] = mn[a];
        const double range = mx[a] - mn[a];
        const double cells = range / cutoff;
        if (!isfinite(range) || range < 0.0 || !isfinite(cells) || cells > 2147483647.0) {
            set_error(err, errlen, "neighbor cell-grid dimension exceeds integer range");
            return 0;
        }
        g->dims[a] = (int)cells < 1 ? 1 : (int)cells;
        const double even = range / g->dims[a];
        g->spacing[a] = cutoff > even ? cutoff : even;
    }
    const int64_t cell_count = (int64_t)g->dims[0] * g->dims[1] * g->dims[2];
    if (cell_count > ((int64_t)1 << 34)) {
        set_error(err, errlen, "neighbor cell-grid is too large");
        return 0;
    }
    int64_t* counts = (int64_t*)calloc((size_t)cell_count, sizeof(int64_t));
    g->offsets = (int64_t*)calloc((size_t)cell_count + 1, sizeof(int64_t));
    g->atoms = (int32_t*)malloc((size_t)n_ext * sizeof(int32_t));
    int64_t* fill = (int64_t*)calloc((size_t)cell_count, sizeof(int64_t));
    int64_t* cell_of = (int64_t*)malloc((size_t)n_ext * sizeof(int64_t));
    if (!counts || !g->offsets || !g->atoms || !fill || !cell_of) {
        free(counts); free(fill); free(cell_of);
        set_error(err, errlen, "out of memory");
        return 0;
    }
    for (int64_t i = 0; i < n_ext; ++i) {
        cell_of[i] = grid_index(g, grid_coordinate(g, ext[i].pos[0], 0),
                                grid_coordinate(g, ext[i].pos[1], 1),
                                grid_coordinate(g, ext[i].pos[2], 2));
        counts[cell_of[i]]++;
    }
    for (int64_t c = 0; c < cell_count; ++c) g->offsets[c + 1] = g->offsets[c] + counts[c];
    for (int64_t i = 0; i < n_ext; ++i) {
        const int64_t c = cell_of[i];
        g->atoms[g->offsets[c] + fill[c]++] = (int32_t)i;
    }
    free(counts);
    free(fill);
    free(cell_of);
    return 1;
}

static void free_grid(cell_grid* g) {
    free(g->offsets);
    free(g->atoms);
    g->offsets = NULL;
    g->atoms = NULL;
}

typedef struct {
    int64_t count, capacity;
    int32_t* atoms;
    int32_t* shifts;
    double* disp;
    double* d2;
} pair_buffer;

static int pair_push(pair_buffer* b, int32_t atom, const int32_t* shift, const double* disp, double d2) {
    if (b->count == b->capacity) {
        const int64_t cap = b->capacity ? b->capacity * 2 : 256;
        int32_t* na = (int32_t*)realloc(b->atoms, (size_t)cap * sizeof(int32_t));
        if (na) b->atoms = na;
        int32_t* ns = (int32_t*)realloc(b->shifts, (size_t)cap * 3 * sizeof(int32_t));
        if (ns) b->shifts = ns;
        double* nd = (double*)realloc(b->disp, (size_t)cap * 3 * sizeof(double));
        if (nd) b->disp = nd;
        double* n2 = (double*)realloc(b->d2, (size_t)cap * sizeof(double));
        if (n2) b->d2 = n2;
        if (!na || !ns || !nd || !n2) return 0;
        b->capacity = cap;
    }
    const int64_t i = b->count++;
    b->atoms[i] = atom;
    b->shifts[i * 3 + 0] = shift[0];
    b->shifts[i * 3 + 1] = shift[1];
    b->shifts[i * 3 + 2] = shift[2];
    b->disp[i * 3 + 0] = disp[0];
    b->disp[i * 3 + 1] = disp[1];
    b->disp[i * 3 + 2] = disp[2];
    b->d2[i] = d2;
    return 1;
}

static void pair_free(pair_buffer* b) {
    free(b->atoms);
    free(b->shifts);
    free(b->disp);
    free(b->d2);
    memset(b, 0, sizeof(*b));
}

/*
 * Graph of one structure.  Atom indices are those of the batch passed in
 * (global indices for a multi-structure batch, neighbor.cpp:475-497).
 * offsets[local] / offsets[local+1] delimit the rows of centre `local`.
 * Candidates are visited in the reference order: 3x3x3 cells z-major, then y,
 * then x, and extended order inside a cell (neighbor.cpp:558-574).
 */
static int build_structure_graph(const double* positions, const double* cell, const int32_t* pbc,
                                 int64_t begin, int64_t end, double cutoff, int include_boundary,
                                 int64_t* offsets_out, pair_buffer* pairs, char* err, int errlen) {
    const int64_t n = end - begin;
    const int periodic = pbc[0] == 1 && pbc[1] == 1 && pbc[2] == 1;
    int bounds[3] = {0, 0, 0};
    if (periodic) {
        double inv[9];
        if (!inverse3(cell, inv)) {
            set_error(err, errlen, "cell matrix is singular");
            return 0;
        }
        for (int a = 0; a < 3; ++a) {
            const double norm = sqrt(inv[0 * 3 + a] * inv[0 * 3 + a] + inv[1 * 3 + a] * inv[1 * 3 + a]
                                     + inv[2 * 3 + a] * inv[2 * 3 + a]);
            const double bound = floor(cutoff * norm + 1.0);
            if (!isfinite(bound) || bound < 0.0 || bound > 2147483647.0) {
                set_error(err, errlen, "periodic image range exceeds integer range");
                return 0;
            }
            bounds[a] = (int)bound;
        }
    }
    const int64_t images = (int64_t)(2 * bounds[0] + 1) * (2 * bounds[1] + 1) * (2 * bounds[2] + 1);
    const int64_t n_ext = images * n;
    ext_atom* ext = (ext_atom*)malloc((size_t)(n_ext > 0 ? n_ext : 1) * sizeof(ext_atom));
    if (!ext) {
        set_error(err, errlen, "out of memory");
        return 0;
    }
    int64_t e = 0;
    /* extended list, neighbor.cpp:471-529: n0 outer, n2 inner, atoms innermost */
    for (int n0 = -bounds[0]; n0 <= bounds[0]; ++n0) {
        for (int n1 = -bounds[1]; n1 <= bounds[1]; ++n1) {
            for (int n2 = -bounds[2]; n2 <= bounds[2]; ++n2) {
                double shift[3];
                for (int a = 0; a < 3; ++a) {
                    shift[a] = ((double)n0 * cell[0 * 3 + a] + (double)n1 * cell[1 * 3 + a])
                        + (double)n2 * cell[2 * 3 + a];
                }
                for (int64_t atom = begin; atom < end; ++atom) {
                    ext[e].atom = (int32_t)atom;
                    ext[e].shift[0] = n0;
                    ext[e].shift[1] = n1;
                    ext[e].shift[2] = n2;
                    for (int a = 0; a < 3; ++a) ext[e].pos[a] = positions[atom * 3 + a] + shift[a];
                    ++e;
                }
            }
        }
    }
    cell_grid grid;
    if (!build_grid(ext, n_ext, cutoff, &grid, err, errlen)) {
        free(ext);
        free_grid(&grid);
        return 0;
    }
    const double cutoff2 = cutoff * cutoff;
    for (int64_t local = 0; local < n; ++local) {
        offsets_out[local] = pairs->count;
        const double* c = positions + (begin + local) * 3;
        const int ix = grid_coordinate(&grid, c[0], 0);
        const int iy = grid_coordinate(&grid, c[1], 1);
        const int iz = grid_coordinate(&grid, c[2], 2);
        for (int z = iz - 1 < 0 ? 0 : iz - 1; z <= (iz + 1 < grid.dims[2] - 1 ? iz + 1 : grid.dims[2] - 1); ++z) {
            for (int y = iy - 1 < 0 ? 0 : iy - 1; y <= (iy + 1 < grid.dims[1] - 1 ? iy + 1 : grid.dims[1] - 1); ++y) {
                for (int x = ix - 1 < 0 ? 0 : ix - 1; x <= (ix + 1 < grid.dims[0] - 1 ? ix + 1 : grid.dims[0] - 1); ++x) {
                    const int64_t cidx = grid_index(&grid, x, y, z);
                    for (int64_t o = grid.offsets[cidx]; o < grid.offsets[cidx + 1]; ++o) {
                        const ext_atom* nb = &ext[grid.atoms[o]];
                        double d[3];
                        d[0] = nb->pos[0] - c[0];
                        d[1] = nb->pos[1] - c[1];
                        d[2] = nb->pos[2] - c[2];
                        const double dd = d[0] * d[0] + d[1] * d[1] + d[2] * d[2];
                        const int keep = include_boundary ? dd <= cutoff2 : dd < cutoff2;
                        if (!keep) continue;
                        if (!pair_push(pairs, nb->atom, nb->shift, d, dd)) {
                            free(ext);
                            free_grid(&grid);
                            set_error(err, errlen, "out of memory");
                            return 0;
                        }
                    }
                }
            }
        }
    }
    offsets_out[n] = pairs->count;
    free(ext);
    free_grid(&grid);
    return 1;
}

/* Result of mdxo_graph_build; all arrays malloc'd and owned by the caller. */
typedef struct {
    int64_t atoms_count;
    int64_t pairs;
    int64_t* offsets;
    int32_t* atoms;
    int32_t* shifts;
    double* disp;
    double* d2;
} mdxo_graph;

/* build_neighbor_graph, neighbor.cpp:703-768: per-structure graphs
 * concatenated in structure order, atom indices global to the batch. */
int mdxo_graph_build(const int32_t* numbers, const double* positions, const double* cells,
                     const int32_t* pbc, const int64_t* offsets, int64_t structures, int64_t atoms,
                     double cutoff, int include_boundary, mdxo_graph* out, char* err, int errlen) {
    memset(out, 0, sizeof(*out));
    if (!isfinite(cutoff) || cutoff <= 0.0) {
        set_error(err, errlen, "neighbor cutoff must be finite and positive");
        return MDXO_INVALID;
    }
    if (!validate_batch(numbers, positions, cells, pbc, offsets, structures, atoms, err, errlen)) {
        return MDXO_INVALID;
    }
    out->atoms_count = atoms;
    out->offsets = (int64_t*)calloc((size_t)atoms + 1, sizeof(int64_t));
    if (!out->offsets) return MDXO_NOMEM;
    pair_buffer pairs;
    memset(&pairs, 0, sizeof(pairs));
    for (int64_t s = 0; s < structures; ++s) {
        if (!build_structure_graph(positions, cells + s * 9, pbc + s * 3, offsets[s], offsets[s + 1],
                                   cutoff, include_boundary, out->offsets + offsets[s], &pairs, err,
                                   errlen)) {
            pair_free(&pairs);
            free(out->offsets);
            out->offsets = NULL;
            return MDXO_INVALID;
        }
    }
    out->pairs = pairs.count;
    out->atoms = pairs.atoms;
    out->shifts = pairs.shifts;
    out->disp = pairs.disp;
    out->d2 = pairs.d2;
    return MDXO_OK;
}

void mdxo_graph_free(mdxo_graph* g) {
    free(g->offsets);
    free(g->atoms);
    free(g->shifts);
    free(g->disp);
    free(g->d2);
    memset(g, 0, sizeof(*g));
}

/* ------------------------------------------------------------------------ */
/* NeighborList descriptor, compute_neighbor_list                           */
/* (cpp/src/standalone/neighbor_list.cpp:15-78).                            */
/* ------------------------------------------------------------------------ */

typedef struct {
    int64_t rows;
    int64_t structures;
    double* values;   /* rows x 9: centre, atom, shift a b c, dx dy dz, distance */
    int64_t* offsets; /* structures + 1 */
} mdxo_pair_table;

/* keep_half_neighbor, cpp/include/mdescriptor/detail/neighbor_filter.hpp:18-38 */
static int keep_half_neighbor(int64_t centre, int64_t atom, const int32_t* shift) {
    if (atom != centre) return atom > centre;
    for (int k = 0; k < 3; ++k) {
        if (shift[k] != 0) return shift[k] > 0;
    }
    return 1;
}

/* neighbor_list.cpp:40-47 (exact_self: neighbor.cpp:683-689) */
static int keep_pair(const mdxo_graph* g, int64_t centre, int64_t p, int full, int self_pairs) {
    const int32_t* shift = g->shifts + 3 * p;
    const int64_t atom = g->atoms[p];
    if (!self_pairs && atom == centre && shift[0] == 0 && shift[1] == 0 && shift[2] == 0) return 0;
    if (!full && !keep_half_neighbor(centre, atom, shift)) return 0;
    return 1;
}

int mdxo_neighbor_list(const int32_t* numbers, const double* positions, const double* cells,
                       const int32_t* pbc, const int64_t* offsets, int64_t structures, int64_t atoms,
                       double cutoff, int full_neighbor_list, int self_pairs, mdxo_pair_table* out,
                       char* err, int errlen) {
    memset(out, 0, sizeof(*out));
    mdxo_graph g;
    /* build_neighbor_graph with its defaults: boundary inclusive, shifts stored */
    const int rc = mdxo_graph_build(numbers, positions, cells, pbc, offsets, structures, atoms, cutoff, 1,
                                    &g, err, errlen);
    if (rc != MDXO_OK) return rc;
    int64_t rows = 0;
    for (int64_t c = 0; c < atoms; ++c) {
        for (int64_t p = g.offsets[c]; p < g.offsets[c + 1]; ++p) {
            rows += keep_pair(&g, c, p, full_neighbor_list, self_pairs);
        }
    }
    out->values = (double*)malloc((size_t)(rows * 9 + 1) * sizeof(double));
    out->offsets = (int64_t*)calloc((size_t)structures + 1, sizeof(int64_t));
    if (!out->values || !out->offsets) {
        free(out->values);
        free(out->offsets);
        memset(out, 0, sizeof(*out));
        mdxo_graph_free(&g);
        return MDXO_NOMEM;
    }
    int64_t row = 0;
    for (int64_t s = 0; s < structures; ++s) {
        out->offsets[s] = row;
        for (int64_t c = offsets[s]; c < offsets[s + 1]; ++c) {
            for (int64_t p = g.offsets[c]; p < g.offsets[c + 1]; ++p) {
                if (!keep_pair(&g, c, p, full_neighbor_list, self_pairs)) continue;
                double* r = out->values + 9 * row;
                r[0] = (double)c;
                r[1] = (double)g.atoms[p];
                r[2] = (double)g.shifts[3 * p + 0];
                r[3] = (double)g.shifts[3 * p + 1];
                r[4] = (double)g.shifts[3 * p + 2];
                r[5] = g.disp[3 * p + 0];
                r[6] = g.disp[3 * p + 1];
                r[7] = g.disp[3 * p + 2];
                r[8] = sqrt(fmax(0.0, g.d2[p]));
                ++row;
            }
        }
    }
    out->offsets[structures] = row;
    out->rows = rows;
    out->structures = structures;
    mdxo_graph_free(&g);
    return MDXO_OK;
}

void mdxo_pair_table_free(mdxo_pair_table* t) {
    free(t->values);
    free(t->offsets);
    memset(t, 0, sizeof(*t));
}

/* ------------------------------------------------------------------------ */
/* Real regular solid harmonics r^l Y_lm.                                   */
/* Layout (soap.cpp:60-69): index l*l + l holds m = 0; l*l + (l-m) holds the */
/* cos part and l*l + (l+m) the sin part, both scaled by sqrt(2).  Values    */
/* follow the Cartesian recurrence of soap.cpp:166-216, which for every l is */
/* the same polynomial as the literal (l<=4, l=6) and Legendre (l>6)         */
/* branches of soap.cpp:101-370 (Condon-Shortley phase included).            */
/* ------------------------------------------------------------------------ */
#define MDXO_LMAX 20

/* solid_harmonic_normalization, soap.cpp:26-38 */
static void harmonic_normalization(int l_max, double* out /* (l_max+1)^2 */) {
    const int width = l_max + 1;
    for (int l = 0; l <= l_max; ++l) {
        for (int m = 0; m <= l; ++m) {
            out[l * width + m] = sqrt((2.0 * l + 1.0) / (4.0 * MDXO_PI)
                                      * exp(lgamma(l - m + 1.0) - lgamma(l + m + 1.0)));
        }
        for (int m = l + 1; m < width; ++m) out[l * width + m] = 0.0;
    }
}

void mdxo_solid_harmonics(double x, double y, double z, int l_max, double* result) {
    double norm[(MDXO_LMAX + 1) * (MDXO_LMAX + 1)];
    double re[MDXO_LMAX + 1][MDXO_LMAX + 1];
    double im[MDXO_LMAX + 1][MDXO_LMAX + 1];
    const int width = l_max + 1;
    harmonic_normalization(l_max, norm);
    const double r2 = x * x + y * y + z * z;
    memset(re, 0, sizeof(re));
    memset(im, 0, sizeof(im));
    re[0][0] = 1.0;
    for (int m = 0; m <= l_max; ++m) {
        if (m > 0) {
            const double f = -(2.0 * m - 1.0);
            re[m][m] = f * (x * re[m - 1][m - 1] - y * im[m - 1][m - 1]);
            im[m][m] = f * (x * im[m - 1][m - 1] + y * re[m - 1][m - 1]);
        }
        if (m < l_max) {
            re[m + 1][m] = (2.0 * m + 1.0) * z * re[m][m];
            im[m + 1][m] = (2.0 * m + 1.0) * z * im[m][m];
        }
        for (int l = m + 2; l <= l_max; ++l) {
            re[l][m] = ((2.0 * l - 1.0) * z * re[l - 1][m] - (l + m - 1.0) * r2 * re[l - 2][m]) / (l - m);
            im[l][m] = ((2.0 * l - 1.0) * z * im[l - 1][m] - (l + m - 1.0) * r2 * im[l - 2][m]) / (l - m);
        }
    }
    for (int l = 0; l <= l_max; ++l) {
        result[l * l + l] = norm[l * width] * re[l][0];
        for (int m = 1; m <= l; ++m) {
            const double f = MDXO_SQRT2 * norm[l * width + m];
            result[l * l + (l - m)] = f * re[l][m];
            result[l * l + (l + m)] = f * im[l][m];
        }
    }
}

/* ------------------------------------------------------------------------ */
/* SOAP: both radial bases, every compression mode and distance weighting.  */
/* Plan: prepare_soap, soap.cpp:507-572.  Expansion: calculate_coefficients */
/* soap.cpp:701-931 (weights :799-812, polynomial :813-863, GTO :864-930).  */
/* Power spectrum: soap.cpp:933-1017.  Averaging: soap.cpp:1019-1142.       */
/* Driver: compute_soap, soap.cpp:1149-1246.                                */
/* ------------------------------------------------------------------------ */

/* Options beyond the GTO/off/unweighted default, the fields of SoapOptions
 * (cpp/include/mdescriptor/descriptor.hpp:17-43) as SoapKernel._ensure_native
 * fills them (core.py:229-270).  A NULL pointer means the defaults. */
typedef struct {
    int32_t weighting_function; /* 0 none, 1 poly, 2 pow, 3 exp */
    int32_t weighting_has_w0;
    double weighting_r0, weighting_c, weighting_d, weighting_m, weighting_w0;
    const double* species_weights; /* [S], NULL = all 1 */
    int32_t compression;           /* 0 off, 1 mu2, 2 mu1nu1, 3 crossover */
    int32_t radial_basis;          /* 0 GTO (alphas, betas), 1 polynomial */
    int32_t grid_size;
    const double* radial_grid;     /* [grid_size] */
    const double* radial_weights;  /* [grid_size] */
    const double* radial_values;   /* [n * grid_size] */
} mdxo_soap_options;

typedef struct {
    int S, n, l_max, L, H, types; /* types: coefficient species (1 for mu2) */
    int64_t coeff_size, features;
    double eta, soap_scale;
    double* power_prefactors;  /* [L] */
    double* radial_prefactors; /* [L*n] */
    double* radial_exponents;  /* [L*n] */
    const double* betas;       /* [L*n*n], index (l*n + n')*n + k */
    double* weighted_qn;       /* polynomial: [Q*n] = w_q r_q^2 values[n][q] */
    mdxo_soap_options opt;
    double species_weights[256];
} soap_plan;

/* soap_features, soap.cpp:373-387 */
static int64_t soap_feature_count(int S, int n, int l_max, int compression) {
    const int64_t L = l_max + 1;
    switch (compression) {
    case 1:
        return (int64_t)n * (n + 1) / 2 * L;
    case 2:
        return (int64_t)S * n * n * L;
    case 3:
        return (int64_t)S * n * (n + 1) / 2 * L;
    default: {
        const int64_t w = (int64_t)S * n;
        return w * (w + 1) / 2 * L;
    }
    }
}

int64_t mdxo_soap_feature_count(int S, int n, int l_max) { return soap_feature_count(S, n, l_max, 0); }

int64_t mdxo_soap_feature_count_ex(int S, int n, int l_max, int compression) {
    return soap_feature_count(S, n, l_max, compression);
}

/* soap_weight, soap.cpp:389-420 */
static double soap_weight(const soap_plan* p, double distance, int exact_self, int type) {
    const mdxo_soap_options* o = &p->opt;
    double value = 1.0;
    if (o->weighting_function != 0) {
        const double ratio = distance / o->weighting_r0;
        switch (o->weighting_function) {
        case 1:
            value = distance > o->weighting_r0
                ? 0.0
                : o->weighting_c * pow(1.0 + 2.0 * ratio * ratio * ratio - 3.0 * ratio * ratio, o->weighting_m);
            break;
        case 2:
            value = o->weighting_c / (o->weighting_d + pow(ratio, o->weighting_m));
            break;
        default:
            value = o->weighting_c / (o->weighting_d + exp(-ratio));
            break;
        }
    }
    if (exact_self && o->weighting_has_w0) value = o->weighting_w0;
    return value * p->species_weights[type];
}

/* polynomial_flir, soap.cpp:450-492 (without the reference's distance cache,
 * which returns the same values) */
static void polynomial_flir(const soap_plan* p, double radius, double* values /* [L*Q] */) {
    const int Q = p->opt.grid_size;
    memset(values, 0, (size_t)p->L * Q * sizeof(double));
    for (int q = 0; q < Q; ++q) {
        const double radial = p->opt.radial_grid[q];
        const double radial2 = radial * radial;
        if (radius <= 1e-14) {
            values[q] = exp(-p->eta * radial2);
            continue;
        }
        const double prefactor = 0.25 / (p->eta * radius * radial);
        const double minus = exp(-p->eta * (radial - radius) * (radial - radius));
        const double plus = exp(-p->eta * (radial + radius) * (radial + radius));
        values[q] = prefactor * (minus - plus);
        if (p->l_max >= 1) values[Q + q] = prefactor * (minus + plus - 2.0 * values[q]);
        for (int l = 2; l <= p->l_max; ++l) {
            const double v = values[(l - 2) * Q + q] - prefactor * (4.0 * l - 2.0) * values[(l - 1) * Q + q];
            values[l * Q + q] = v > 0.0 ? v : 0.0;
        }
    }
}

typedef struct {
    double* coeff;
    double* harm;    /* [H * count] */
    int64_t* order;  /* [count] graph index in species order */
    double* hsum;    /* [2 l_max + 1] */
    double* ylm;     /* [H] */
    double* power;   /* [F] */
    double* weight;  /* [count] */
    double* flir;    /* polynomial: [L * Q] */
    double* integrand; /* polynomial: [types * H * Q] */
    double* summed;  /* mu1nu1: [n * H] */
    int64_t capacity;
} centre_workspace;

static void compute_centre_coefficients(const soap_plan* p, const int32_t* atom_type, int64_t centre,
                                        const int64_t* graph_offsets, const int32_t* graph_atoms,
                                        const int32_t* graph_shifts, const double* graph_disp,
                                        const double* graph_d2, centre_workspace* w) {
    const int64_t begin = graph_offsets[centre];
    const int64_t count = graph_offsets[centre + 1] - begin;
    double* coeff = w->coeff;
    memset(coeff, 0, (size_t)p->coeff_size * sizeof(double));
    /* neighbour order: mu2 and one species keep the graph order, otherwise a
     * stable counting sort by species (soap.cpp:727-760) */
    int64_t type_offsets[257];
    int64_t cursor[256];
    if (p->opt.compression == 1 || p->S == 1) {
        type_offsets[0] = 0;
        type_offsets[1] = count;
        for (int64_t i = 0; i < count; ++i) w->order[i] = begin + i;
    } else {
        memset(cursor, 0, sizeof(cursor));
        for (int64_t i = 0; i < count; ++i) cursor[atom_type[graph_atoms[begin + i]]]++;
        type_offsets[0] = 0;
        for (int t = 0; t < p->S; ++t) {
            type_offsets[t + 1] = type_offsets[t] + cursor[t];
            cursor[t] = type_offsets[t];
        }
        for (int64_t i = 0; i < count; ++i) {
            const int t = atom_type[graph_atoms[begin + i]];
            w->order[cursor[t]++] = begin + i;
        }
    }
    /* harmonics, SoA [h * count + j], soap.cpp:761-780 */
    for (int64_t j = 0; j < count; ++j) {
        const int64_t src = w->order[j];
        mdxo_solid_harmonics(graph_disp[src * 3 + 0], graph_disp[src * 3 + 1], graph_disp[src * 3 + 2],
                             p->l_max, w->ylm);
        for (int h = 0; h < p->H; ++h) w->harm[(int64_t)h * count + j] = w->ylm[h];
    }
    /* weights, soap.cpp:781-812: the neighbour's own species under mu2, the
     * species run otherwise (the same thing once sorted) */
    for (int64_t j = 0; j < count; ++j) {
        const int64_t src = w->order[j];
        const int32_t atom = graph_atoms[src];
        const int exact_self = atom == centre && graph_shifts[src * 3] == 0 && graph_shifts[src * 3 + 1] == 0
            && graph_shifts[src * 3 + 2] == 0;
        const int type = (p->opt.compression == 1 || p->S > 1) ? atom_type[atom] : 0;
        w->weight[j] = soap_weight(p, sqrt(graph_d2[src]), exact_self, type);
    }
    if (p->opt.radial_basis == 1) {
        /* polynomial basis, soap.cpp:813-863 */
        const int Q = p->opt.grid_size;
        const int64_t stride = (int64_t)p->H * Q;
        memset(w->integrand, 0, (size_t)(p->types * stride) * sizeof(double));
        for (int t = 0; t < p->types; ++t) {
            const int64_t tb = p->opt.compression == 1 ? 0 : type_offsets[t];
            const int64_t te = p->opt.compression == 1 ? count : type_offsets[t + 1];
            for (int64_t j = tb; j < te; ++j) {
                const double radius = sqrt(graph_d2[w->order[j]]);
                polynomial_flir(p, radius, w->flir);
                const double inverse_radius = radius <= 1e-14 ? 0.0 : 1.0 / radius;
                double inverse_radius_power = 1.0;
                for (int l = 0; l <= p->l_max; ++l) {
                    const double scale = radius <= 1e-14 ? (l == 0 ? 4.0 * MDXO_PI * w->weight[j] : 0.0)
                                                         : 4.0 * MDXO_PI * inverse_radius_power * w->weight[j];
                    const double* source = w->flir + (int64_t)l * Q;
                    for (int m = 0; m < 2 * l + 1; ++m) {
                        const double factor = scale * w->harm[(int64_t)(l * l + m) * count + j];
                        double* target = w->integrand + t * stride + (int64_t)(l * l + m) * Q;
                        for (int q = 0; q < Q; ++q) target[q] += factor * source[q];
                    }
                    inverse_radius_power *= inverse_radius;
                }
            }
        }
        for (int t = 0; t < p->types; ++t) {
            for (int l = 0; l <= p->l_max; ++l) {
                for (int nn = 0; nn < p->n; ++nn) {
                    double* dst = coeff + ((int64_t)t * p->n + nn) * p->H + l * l;
                    for (int m = 0; m < 2 * l + 1; ++m) {
                        const double* integrand = w->integrand + t * stride + (int64_t)(l * l + m) * Q;
                        double sum = 0.0;
                        for (int q = 0; q < Q; ++q) sum += integrand[q] * p->weighted_qn[(int64_t)q * p->n + nn];
                        dst[m] += sum;
                    }
                }
            }
        }
        return;
    }
    /* GTO: accumulate per species, l, k then fold beta, soap.cpp:864-929 */
    for (int t = 0; t < p->types; ++t) {
        const int64_t tb = p->opt.compression == 1 ? 0 : type_offsets[t];
        const int64_t te = p->opt.compression == 1 ? count : type_offsets[t + 1];
        for (int l = 0; l <= p->l_max; ++l) {
            const int mc = 2 * l + 1;
            for (int k = 0; k < p->n; ++k) {
                const int ri = l * p->n + k;
                const double pref = p->radial_prefactors[ri];
                const double expo = p->radial_exponents[ri];
                for (int m = 0; m < mc; ++m) w->hsum[m] = 0.0;
                for (int64_t j = tb; j < te; ++j) {
                    const double radial = pref * exp(-expo * graph_d2[w->order[j]]);
                    for (int m = 0; m < mc; ++m) {
                        w->hsum[m] += radial * w->harm[(int64_t)(l * l + m) * count + j] * w->weight[j];
                    }
                }
                for (int nn = 0; nn < p->n; ++nn) {
                    const double beta = p->betas[(l * p->n + nn) * p->n + k];
                    double* dst = coeff + ((int64_t)t * p->n + nn) * p->H + l * l;
                    for (int m = 0; m < mc; ++m) dst[m] += p->soap_scale * beta * w->hsum[m];
                }
            }
        }
    }
}

static double dot_channels(const double* a, const double* b, int l) {
    double sum = 0.0;
    for (int m = 0; m < 2 * l + 1; ++m) sum += a[l * l + m] * b[l * l + m];
    return sum;
}

/* power_spectrum, soap.cpp:933-1017; summed [n * H] is scratch for mu1nu1 */
static void power_spectrum(const soap_plan* p, const double* c, double* summed, double* out) {
    int64_t f = 0;
    const int64_t H = p->H;
    const int n = p->n;
    if (p->opt.compression == 1) {
        for (int l = 0; l <= p->l_max; ++l) {
            for (int n1 = 0; n1 < n; ++n1) {
                for (int n2 = n1; n2 < n; ++n2) {
                    out[f++] = p->power_prefactors[l] * dot_channels(c + n1 * H, c + n2 * H, l);
                }
            }
        }
    } else if (p->opt.compression == 2) {
        memset(summed, 0, (size_t)(n * H) * sizeof(double));
        for (int t = 0; t < p->S; ++t) {
            for (int nn = 0; nn < n; ++nn) {
                for (int64_t i = 0; i < H; ++i) summed[nn * H + i] += c[((int64_t)t * n + nn) * H + i];
            }
        }
        for (int t = 0; t < p->S; ++t) {
            for (int l = 0; l <= p->l_max; ++l) {
                for (int n1 = 0; n1 < n; ++n1) {
                    for (int n2 = 0; n2 < n; ++n2) {
                        out[f++] = p->power_prefactors[l]
                            * dot_channels(c + ((int64_t)t * n + n1) * H, summed + n2 * H, l);
                    }
                }
            }
        }
    } else if (p->opt.compression == 3) {
        for (int t = 0; t < p->S; ++t) {
            for (int l = 0; l <= p->l_max; ++l) {
                for (int n1 = 0; n1 < n; ++n1) {
                    for (int n2 = n1; n2 < n; ++n2) {
                        out[f++] = p->power_prefactors[l]
                            * dot_channels(c + ((int64_t)t * n + n1) * H, c + ((int64_t)t * n + n2) * H, l);
                    }
                }
            }
        }
    } else {
        for (int t1 = 0; t1 < p->S; ++t1) {
            for (int t2 = t1; t2 < p->S; ++t2) {
                for (int l = 0; l <= p->l_max; ++l) {
                    for (int n1 = 0; n1 < n; ++n1) {
                        for (int n2 = (t1 == t2 ? n1 : 0); n2 < n; ++n2) {
                            out[f++] = p->power_prefactors[l]
                                * dot_channels(c + ((int64_t)t1 * n + n1) * H, c + ((int64_t)t2 * n + n2) * H, l);
                        }
                    }
                }
            }
        }
    }
}

static int workspace_reserve(centre_workspace* w, const soap_plan* p, int64_t count) {
    if (w->coeff == NULL) {
        const int Q = p->opt.radial_basis == 1 ? p->opt.grid_size : 0;
        w->coeff = (double*)malloc((size_t)p->coeff_size * sizeof(double));
        w->hsum = (double*)malloc((size_t)(2 * p->l_max + 1) * sizeof(double));
        w->ylm = (double*)malloc((size_t)p->H * sizeof(double));
        w->power = (double*)malloc((size_t)p->features * sizeof(double));
        w->summed = (double*)malloc((size_t)p->n * p->H * sizeof(double));
        w->flir = (double*)malloc((size_t)(p->L * Q + 1) * sizeof(double));
        w->integrand = (double*)malloc((size_t)((int64_t)p->types * p->H * Q + 1) * sizeof(double));
        if (!w->coeff || !w->hsum || !w->ylm || !w->power || !w->summed || !w->flir || !w->integrand) return 0;
    }
    if (count > w->capacity) {
        const int64_t cap = count * 2;
        free(w->harm);
        free(w->order);
        free(w->weight);
        w->harm = (double*)malloc((size_t)cap * p->H * sizeof(double));
        w->order = (int64_t*)malloc((size_t)cap * sizeof(int64_t));
        w->weight = (double*)malloc((size_t)cap * sizeof(double));
        if (!w->harm || !w->order || !w->weight) return 0;
        w->capacity = cap;
    }
    return 1;
}

static void workspace_free(centre_workspace* w) {
    free(w->coeff);
    free(w->harm);
    free(w->order);
    free(w->hsum);
    free(w->ylm);
    free(w->power);
    free(w->weight);
    free(w->flir);
    free(w->integrand);
    free(w->summed);
    memset(w, 0, sizeof(*w));
}

/* compute_soap_structure (soap.cpp:598-1146) for one structure whose graph is
 * given with local atom indices.  parallel != 0 runs centres in an OpenMP
 * loop with per-thread partial sums, as in soap.cpp:1022-1060, 1071-1112. */
static int soap_structure(const soap_plan* p, const int32_t* atom_type, int64_t atom_count,
                          const int64_t* g_off, const int32_t* g_atoms, const int32_t* g_shifts,
                          const double* g_disp, const double* g_d2, int average, int parallel, int threads,
                          double* out, const volatile int32_t* cancel) {
    const int64_t F = p->features;
    const int64_t C = p->coeff_size;
    int failed = 0;
    if (average == 1 || average == 2) {
        const int64_t width = average == 1 ? C : F;
        double* total = (double*)calloc((size_t)width, sizeof(double));
        if (!total) return MDXO_NOMEM;
        const int nt = parallel ? threads : 1;
        double* partial = (double*)calloc((size_t)width * nt, sizeof(double));
        if (!partial) {
            free(total);
            return MDXO_NOMEM;
        }
#pragma omp parallel num_threads(nt) if (parallel)
        {
            int tid = 0;
#ifdef _OPENMP
            tid = omp_get_thread_num();
#endif
            centre_workspace w;
            memset(&w, 0, sizeof(w));
#pragma omp for schedule(static)
            for (int64_t c = 0; c < atom_count; ++c) {
                if (failed || (cancel && *cancel)) continue;
                if (!workspace_reserve(&w, p, g_off[c + 1] - g_off[c])) {
                    failed = 1;
                    continue;
                }
                compute_centre_coefficients(p, atom_type, c, g_off, g_atoms, g_shifts, g_disp, g_d2, &w);
                double* dst = partial + (int64_t)tid * width;
                if (average == 1) {
                    for (int64_t i = 0; i < C; ++i) dst[i] += w.coeff[i];
                } else {
                    power_spectrum(p, w.coeff, w.summed, w.power);
                    for (int64_t i = 0; i < F; ++i) dst[i] += w.power[i];
                }
            }
            workspace_free(&w);
        }
        if (failed) {
            free(total);
            free(partial);
            return MDXO_NOMEM;
        }
        if (cancel && *cancel) {
            free(total);
            free(partial);
            return MDXO_CANCELLED;
        }
        for (int t = 0; t < nt; ++t) {
            for (int64_t i = 0; i < width; ++i) total[i] += partial[(int64_t)t * width + i];
        }
        if (average == 1) {
            if (atom_count > 0) {
                const double inv = 1.0 / (double)atom_count;
                for (int64_t i = 0; i < C; ++i) total[i] *= inv;
            }
            double* summed = (double*)malloc((size_t)p->n * p->H * sizeof(double));
            if (!summed) {
                free(total);
                free(partial);
                return MDXO_NOMEM;
            }
            power_spectrum(p, total, summed, out);
            free(summed);
        } else {
            if (atom_count > 0) {
                const double inv = 1.0 / (double)atom_count;
                for (int64_t i = 0; i < F; ++i) out[i] = total[i] * inv;
            } else {
                for (int64_t i = 0; i < F; ++i) out[i] = 0.0;
            }
        }
        free(total);
        free(partial);
        return MDXO_OK;
    }
#pragma omp parallel num_threads(parallel ? threads : 1) if (parallel)
    {
        centre_workspace w;
        memset(&w, 0, sizeof(w));
#pragma omp for schedule(static)
        for (int64_t c = 0; c < atom_count; ++c) {
            if (failed || (cancel && *cancel)) continue;
            if (!workspace_reserve(&w, p, g_off[c + 1] - g_off[c])) {
                failed = 1;
                continue;
            }
            compute_centre_coefficients(p, atom_type, c, g_off, g_atoms, g_shifts, g_disp, g_d2, &w);
            power_spectrum(p, w.coeff, w.summed, out + c * F);
        }
        workspace_free(&w);
    }
    if (failed) return MDXO_NOMEM;
    if (cancel && *cancel) return MDXO_CANCELLED;
    return MDXO_OK;
}

/*
 * mdxo_soap: compute_soap (soap.cpp:1149-1246).  average: 0 off, 1 inner,
 * 2 outer.  `output` is caller-allocated C-order f64 [rows, features], rows =
 * structures when averaging, else atoms.  alphas [L*n] and betas [L*n*n] (GTO)
 * or the polynomial grid/weights/values in `options` are supplied by the
 * caller exactly as the reference passes them (core.py:237-245).  options may
 * be NULL (GTO, compression off, no weighting, unit species weights).
 * decomposition: 0 = the reference's (one structure: centre-parallel;
 * several: structure-parallel with serial centres, soap.cpp:1218-1245);
 * 1 = every structure centre-parallel over all threads.
 */
static int all_finite(const double* v, int64_t count) {
    for (int64_t i = 0; i < count; ++i) {
        if (!isfinite(v[i])) return 0;
    }
    return 1;
}

int mdxo_soap(const int32_t* numbers, const double* positions, const double* cells, const int32_t* pbc,
              const int64_t* offsets, int64_t structures, int64_t atoms, const int32_t* species, int S,
              int n_max, int l_max, double r_cut, double sigma, const double* alphas, const double* betas,
              const mdxo_soap_options* options, int average, int num_threads, int decomposition,
              double* output, const volatile int32_t* cancel, char* err, int errlen) {
    if (!validate_batch(numbers, positions, cells, pbc, offsets, structures, atoms, err, errlen)) {
        return MDXO_INVALID;
    }
    soap_plan p;
    memset(&p, 0, sizeof(p));
    if (options != NULL) p.opt = *options;
    /* parameter checks of compute_soap, soap.cpp:1150-1210, in its order */
    if (S < 1 || S > 256 || !isfinite(r_cut) || !isfinite(sigma) || r_cut <= 0.0 || sigma <= 0.0
        || n_max < 1 || l_max < 0 || l_max > MDXO_LMAX || average < 0 || average > 2 || p.opt.radial_basis < 0
        || p.opt.radial_basis > 1 || p.opt.compression < 0 || p.opt.compression > 3) {
        set_error(err, errlen, "invalid SOAP parameters");
        return MDXO_INVALID;
    }
    if (p.opt.radial_basis == 0) {
        if (alphas == NULL || betas == NULL) {
            set_error(err, errlen, "invalid SOAP radial basis size");
            return MDXO_INVALID;
        }
    } else if (p.opt.grid_size < 2 || p.opt.radial_grid == NULL || p.opt.radial_weights == NULL
               || p.opt.radial_values == NULL) {
        set_error(err, errlen, "invalid SOAP polynomial radial basis size");
        return MDXO_INVALID;
    }
    if (p.opt.radial_basis == 0
        && (!all_finite(alphas, (int64_t)(l_max + 1) * n_max)
            || !all_finite(betas, (int64_t)(l_max + 1) * n_max * n_max))) {
        set_error(err, errlen, "SOAP radial basis must be finite");
        return MDXO_INVALID;
    }
    if (p.opt.radial_basis == 1) {
        for (int q = 0; q < p.opt.grid_size; ++q) {
            const double v = p.opt.radial_grid[q];
            if (!isfinite(v) || v < 0.0 || v > r_cut) {
                set_error(err, errlen, "SOAP polynomial radial grid must be finite and in range");
                return MDXO_INVALID;
            }
        }
        for (int q = 0; q < p.opt.grid_size; ++q) {
            const double v = p.opt.radial_weights[q];
            if (!isfinite(v) || v <= 0.0) {
                set_error(err, errlen, "SOAP polynomial radial weights must be positive and finite");
                return MDXO_INVALID;
            }
        }
        if (!all_finite(p.opt.radial_values, (int64_t)n_max * p.opt.grid_size)) {
            set_error(err, errlen, "SOAP polynomial radial basis must be finite");
            return MDXO_INVALID;
        }
    }
    for (int t = 0; t < S; ++t) {
        p.species_weights[t] = p.opt.species_weights != NULL ? p.opt.species_weights[t] : 1.0;
    }
    if (!all_finite(p.species_weights, S)) {
        set_error(err, errlen, "SOAP species weights must be finite");
        return MDXO_INVALID;
    }
    if (p.opt.weighting_function != 0) {
        if (p.opt.weighting_function < 1 || p.opt.weighting_function > 3 || !isfinite(p.opt.weighting_r0)
            || p.opt.weighting_r0 <= 0.0 || !isfinite(p.opt.weighting_c) || p.opt.weighting_c < 0.0
            || !isfinite(p.opt.weighting_d) || p.opt.weighting_d < 0.0 || !isfinite(p.opt.weighting_m)
            || p.opt.weighting_m < 0.0) {
            set_error(err, errlen, "invalid SOAP weighting parameters");
            return MDXO_INVALID;
        }
    }
    if (p.opt.weighting_has_w0 && (!isfinite(p.opt.weighting_w0) || p.opt.weighting_w0 < 0.0)) {
        set_error(err, errlen, "invalid SOAP w0 weighting");
        return MDXO_INVALID;
    }
    p.S = S;
    p.n = n_max;
    p.l_max = l_max;
    p.L = l_max + 1;
    p.H = p.L * p.L;
    p.types = p.opt.compression == 1 ? 1 : S;
    p.coeff_size = (int64_t)p.types * n_max * p.H;
    p.features = soap_feature_count(S, n_max, l_max, p.opt.compression);
    int32_t* atom_type = (int32_t*)malloc((size_t)(atoms > 0 ? atoms : 1) * sizeof(int32_t));
    if (!atom_type) return MDXO_NOMEM;
    for (int64_t i = 0; i < atoms; ++i) {
        int found = -1;
        for (int t = 0; t < S; ++t) {
            if (species[t] == numbers[i]) found = t;
        }
        if (found < 0) {
            free(atom_type);
            set_error(err, errlen, "batch contains an atomic number outside calculator species");
            return MDXO_INVALID;
        }
        atom_type[i] = found;
    }
    /* prepare_soap, soap.cpp:507-572 */
    p.eta = 1.0 / (2.0 * sigma * sigma);
    p.soap_scale = MDXO_PI * sqrt(MDXO_PI);
    p.power_prefactors = (double*)malloc((size_t)p.L * sizeof(double));
    p.radial_prefactors = (double*)calloc((size_t)p.L * n_max, sizeof(double));
    p.radial_exponents = (double*)calloc((size_t)p.L * n_max, sizeof(double));
    p.weighted_qn = (double*)calloc((size_t)(p.opt.radial_basis == 1 ? p.opt.grid_size : 1) * n_max, sizeof(double));
    p.betas = betas;
    for (int l = 0; l <= l_max; ++l) p.power_prefactors[l] = MDXO_PI * sqrt(8.0 / (2.0 * l + 1.0));
    if (p.opt.radial_basis == 0) {
        double eta_power = 1.0;
        for (int l = 0; l <= l_max; ++l) {
            if (l > 0) eta_power *= p.eta;
            for (int k = 0; k < n_max; ++k) {
                const int idx = l * n_max + k;
                const double denominator = alphas[idx] + p.eta;
                p.radial_prefactors[idx] = eta_power * pow(denominator, -l - 1.5);
                p.radial_exponents[idx] = alphas[idx] * p.eta / denominator;
            }
        }
    } else {
        for (int q = 0; q < p.opt.grid_size; ++q) {
            const double radial = p.opt.radial_grid[q];
            const double quadrature = p.opt.radial_weights[q] * radial * radial;
            for (int nn = 0; nn < n_max; ++nn) {
                p.weighted_qn[(int64_t)q * n_max + nn] = quadrature * p.opt.radial_values[(int64_t)nn * p.opt.grid_size + q];
            }
        }
    }
    /* graph cutoff padding, soap.cpp:1214 */
    const double padding = sigma * sqrt(-2.0 * log(1e-3));
    const double cutoff = r_cut + padding;
    int threads = num_threads;
#ifdef _OPENMP
    if (threads <= 0) threads = omp_get_max_threads();
#else
    threads = 1;
#endif
    const int64_t F = p.features;
    int status = MDXO_OK;
    const int averaged = average != 0;
    const int structure_parallel = decomposition == 0 && structures > 1;
    int st_threads = threads;
    if (structure_parallel && st_threads > structures) st_threads = (int)structures; /* descriptor_common.hpp:34-38 */
#pragma omp parallel for schedule(static) num_threads(st_threads) if (structure_parallel)
    for (int64_t s = 0; s < structures; ++s) {
        if (status != MDXO_OK || (cancel && *cancel)) continue;
        const int64_t b = offsets[s], e = offsets[s + 1], n = e - b;
        int64_t* g_off = (int64_t*)calloc((size_t)n + 1, sizeof(int64_t));
        pair_buffer pairs;
        memset(&pairs, 0, sizeof(pairs));
        char local_err[256] = {0};
        /* structure_view (extra_common.hpp:36-51): local atom indices */
        int ok = g_off != NULL
            && build_structure_graph(positions + b * 3, cells + s * 9, pbc + s * 3, 0, n, cutoff, 1, g_off,
                                     &pairs, local_err, (int)sizeof(local_err));
        if (!ok) {
#pragma omp critical
            {
                status = MDXO_INVALID;
                set_error(err, errlen, local_err[0] ? local_err : "graph construction failed");
            }
        } else {
            double* dst = output + (averaged ? s : b) * F;
            const int rc = soap_structure(&p, atom_type + b, n, g_off, pairs.atoms, pairs.shifts, pairs.disp,
                                          pairs.d2, average, !structure_parallel, threads, dst, cancel);
            if (rc != MDXO_OK) {
#pragma omp critical
                {
                    status = rc;
                }
            }
        }
        free(g_off);
        pair_free(&pairs);
    }
    if (status == MDXO_OK && cancel && *cancel) status = MDXO_CANCELLED;
    free(atom_type);
    free(p.power_prefactors);
    free(p.radial_prefactors);
    free(p.radial_exponents);
    free(p.weighted_qn);
    return status;
}
