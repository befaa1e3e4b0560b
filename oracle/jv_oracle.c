/*
 * jv_oracle.c -- CPU restatement of torchmatch's float32 `jonker_dense_batch`
 * and `jonker_compact_batch`.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * kernels in torchmatch_amd/csrc; nothing in the product links, loads or
 * calls it.  It is used by tests/, by __graft_entry__.smoke() and by the
 * cpu_baseline leg of bench.py, always as the thing compared against.
 *
 * What it restates (paths relative to the reference repository root,
 * sources/torchmatch/assignment/cpu/):
 *   ops.cpp:67-93            compute_sentinel   -> jvo_sentinel()
 *   ops.cpp:176-289          solve_batch        -> jvo_dense_batch()
 *   jonker_dense_core.cpp:15-60  solve_square_impl -> jvo_square()
 *   jonker_dense_flat.h:27-43    find_dense     -> jvo_find_tied()
 *   jonker_dense_flat.h:45-73    scan_dense     -> jvo_scan()
 *   jonker_dense_flat.h:75-122   find_path_dense-> jvo_path()
 *   jonker_dense_flat.h:124-176  ccrrt_dense    -> jvo_column_reduction()
 *   jonker_dense_flat.h:178-235  carr_dense     -> jvo_row_reduction()
 *   jonker_dense_flat.h:237-258  ca_dense       -> jvo_augment()
 *   jonker_dense_flat.h:260-274  jonker_internal_flat -> jvo_square()
 *   jonker_compact_core.h:20-43  find_umins_regular -> jvoc_two_min()
 *   jonker_compact_core.h:51-252 jonker_compact_kernel -> jvoc_square()
 *   ops.cpp:431-433, jonker_compact_core.h:279-301
 *                                jonker_compact_batch -> jvo_compact_batch()
 *
 * Every float32 expression keeps the reference's operand order and every
 * comparison keeps its strictness, because the int64 row->col mapping must
 * match bit for bit, including on exact ties.  Compile without fast-math.
 *
 * Pinning (see tests/test_oracle_jv.py): the reference core itself, built
 * from its own source by oracle/Makefile into oracle/_ref, on thousands of
 * random / tied / masked problems; scipy.optimize.linear_sum_assignment on
 * the optimal total cost; brute force over permutations for K <= 7; the
 * reference tests' known answers (test_lap_inf_mask.py).
 *
 * Instrumentation: jvo_dense_batch_counted() also returns, per problem, the
 * number of reduced-cost evaluations ("relaxations") each phase performs.
 * That count is the algorithmic work unit the GPU roofline is priced in.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define JVO_LARGE 1e18f /* jonker_dense_flat.h:22-23, LARGE_V<float> */

enum { JVO_OK = 0, JVO_ERR_NAN = 1, JVO_ERR_NEG_INF = 2, JVO_ERR_ALLOC = 3 };

typedef struct {
    int64_t relax;  /* reduced-cost evaluations c[i][j] - v[j] (all phases) */
    int64_t paths;  /* augmenting paths searched in the augmentation phase */
    int64_t scans;  /* rows scanned inside augmenting-path searches */
    int64_t rr_steps; /* steps of the augmenting row reduction (both rounds) */
} jvo_counts;

/* Per-solve scratch, sized K (mirrors the thread-local vectors of
 * jonker_dense_core.cpp:21-36). */
typedef struct {
    int32_t *x, *y, *free_rows, *pred, *cols;
    float *v, *d;
    char *unique;
} jvo_scratch;

/* find_dense (jonker_dense_flat.h:27-43): among cols[lo..n), bring every
 * column whose d equals the running minimum to the front [lo, hi), with a
 * swap-based partition that restarts whenever a strictly smaller d shows up.
 * Returns hi. */
static uint32_t jvo_find_tied(uint32_t n, uint32_t lo, const float *d, int32_t *cols) {
    uint32_t hi = lo + 1;
    float best = d[cols[lo]];
    for (uint32_t k = lo + 1; k < n; ++k) {
        const int32_t j = cols[k];
        const float dj = d[j];
        if (!(dj <= best))
            continue;
        if (dj < best) {
            best = dj;
            hi = lo;
        }
        cols[k] = cols[hi];
        cols[hi] = j;
        ++hi;
    }
    return hi;
}

/* scan_dense (jonker_dense_flat.h:45-73).  Pops the tied columns one by one,
 * relaxes every not-yet-tied column through the row that owns the popped
 * column, and returns the first unassigned column that becomes tied at the
 * current minimum.  On that early return *plo / *phi are left untouched. */
static int32_t jvo_scan(uint32_t n, const float *c, uint32_t *plo, uint32_t *phi,
                        float *d, int32_t *cols, int32_t *pred, const int32_t *y,
                        const float *v, jvo_counts *cnt) {
    uint32_t lo = *plo, hi = *phi;
    while (lo != hi) {
        const int32_t jp = cols[lo];
        ++lo;
        const int32_t i = y[jp];
        const float level = d[jp];
        const float *row = c + (size_t)i * n;
        const float h = row[jp] - v[jp] - level;
        if (cnt) {
            cnt->scans++;
            cnt->relax += 1 + (int64_t)(n - hi);
        }
        for (uint32_t k = hi; k < n; ++k) {
            const int32_t j = cols[k];
            const float r = row[j] - v[j] - h;
            if (!(r < d[j]))
                continue;
            d[j] = r;
            pred[j] = i;
            if (r == level) {
                if (y[j] < 0)
                    return j;
                cols[k] = cols[hi];
                cols[hi] = j;
                ++hi;
            }
        }
    }
    *plo = lo;
    *phi = hi;
    return -1;
}

/* find_path_dense (jonker_dense_flat.h:75-122): Dijkstra over reduced costs
 * from free row `start`.  Returns the unassigned column the path ends at and
 * applies the dual update to the columns made ready before the last level. */
static int32_t jvo_path(uint32_t n, const float *c, int32_t start, const int32_t *y,
                        float *v, int32_t *pred, int32_t *cols, float *d,
                        jvo_counts *cnt) {
    uint32_t lo = 0, hi = 0, n_ready = 0;
    int32_t final_j = -1;
    const float *row = c + (size_t)start * n;
    for (uint32_t j = 0; j < n; ++j) {
        cols[j] = (int32_t)j;
        d[j] = row[j] - v[j];
        pred[j] = start;
    }
    if (cnt) {
        cnt->paths++;
        cnt->relax += n;
    }
    while (final_j < 0) {
        if (lo == hi) {
            n_ready = lo;
            hi = jvo_find_tied(n, lo, d, cols);
            /* the LAST unassigned column of the tied block wins (no break,
             * jonker_dense_flat.h:107-110) */
            for (uint32_t k = lo; k < hi; ++k)
                if (y[cols[k]] < 0)
                    final_j = cols[k];
        }
        if (final_j < 0)
            final_j = jvo_scan(n, c, &lo, &hi, d, cols, pred, y, v, cnt);
    }
    const float level = d[cols[lo]];
    for (uint32_t k = 0; k < n_ready; ++k) {
        const int32_t j = cols[k];
        v[j] += d[j] - level;
    }
    return final_j;
}

/* ccrrt_dense (jonker_dense_flat.h:124-176): column reduction, reverse-order
 * greedy assignment and reduction transfer.  Returns the number of free rows
 * written to free_rows. */
static int32_t jvo_column_reduction(uint32_t n, const float *c, jvo_scratch *s,
                                    jvo_counts *cnt) {
    int32_t *x = s->x, *y = s->y, *fr = s->free_rows;
    float *v = s->v;
    char *unique = s->unique;
    for (uint32_t k = 0; k < n; ++k) {
        unique[k] = 1;
        x[k] = -1;
        v[k] = JVO_LARGE;
        y[k] = 0;
    }
    /* column minima; strict '<' keeps the lowest row on ties */
    for (uint32_t i = 0; i < n; ++i) {
        const float *row = c + (size_t)i * n;
        for (uint32_t j = 0; j < n; ++j)
            if (row[j] < v[j]) {
                v[j] = row[j];
                y[j] = (int32_t)i;
            }
    }
    /* columns in decreasing order: the first (highest) column claiming a row
     * keeps it, later claimants are dropped and the row is marked shared */
    for (int32_t j = (int32_t)n - 1; j >= 0; --j) {
        const int32_t i = y[j];
        if (x[i] < 0) {
            x[i] = j;
        } else {
            unique[i] = 0;
            y[j] = -1;
        }
    }
    int32_t n_free = 0;
    for (uint32_t i = 0; i < n; ++i) {
        if (x[i] < 0) {
            fr[n_free++] = (int32_t)i;
            continue;
        }
        if (!unique[i])
            continue;
        const int32_t own = x[i];
        const float *row = c + (size_t)i * n;
        float mn = JVO_LARGE;
        for (uint32_t j = 0; j < n; ++j) {
            if ((int32_t)j == own)
                continue;
            const float r = row[j] - v[j];
            if (r < mn)
                mn = r;
        }
        if (cnt)
            cnt->relax += n - 1;
        v[own] -= mn;
    }
    if (cnt)
        cnt->relax += (int64_t)n * n;
    return n_free;
}

/* carr_dense (jonker_dense_flat.h:178-235): augmenting row reduction over the
 * free rows.  Returns the number of rows still free afterwards. */
static int32_t jvo_row_reduction(uint32_t n, const float *c, uint32_t n_free,
                                 jvo_scratch *s, jvo_counts *cnt) {
    int32_t *x = s->x, *y = s->y, *fr = s->free_rows;
    float *v = s->v;
    uint32_t cur = 0, rounds = 0;
    int32_t still_free = 0;
    while (cur < n_free) {
        ++rounds;
        const int32_t fi = fr[cur++];
        const float *row = c + (size_t)fi * n;
        /* lowest and second-lowest reduced cost of the row, first index wins
         * ties; the second slot starts at (LARGE, -1) */
        int32_t j1 = 0, j2 = -1;
        float u1 = row[0] - v[0], u2 = JVO_LARGE;
        for (uint32_t j = 1; j < n; ++j) {
            const float r = row[j] - v[j];
            if (!(r < u2))
                continue;
            if (r >= u1) {
                u2 = r;
                j2 = (int32_t)j;
            } else {
                u2 = u1;
                j2 = j1;
                u1 = r;
                j1 = (int32_t)j;
            }
        }
        if (cnt) {
            cnt->relax += n;
            cnt->rr_steps += 1;
        }
        int32_t i0 = y[j1];
        const float lowered = v[j1] - (u2 - u1);
        const int lowers = lowered < v[j1];
        if (rounds < cur * n) {
            if (lowers) {
                v[j1] = lowered;
            } else if (i0 >= 0 && j2 >= 0) {
                j1 = j2;
                i0 = y[j2];
            }
            if (i0 >= 0) {
                if (lowers)
                    fr[--cur] = i0;
                else
                    fr[still_free++] = i0;
            }
        } else if (i0 >= 0) {
            fr[still_free++] = i0;
        }
        x[fi] = j1;
        y[j1] = fi;
    }
    return still_free;
}

/* ca_dense (jonker_dense_flat.h:237-258): one augmenting path per remaining
 * free row, then flip the assignment along the predecessor chain (at most n
 * steps). */
static void jvo_augment(uint32_t n, const float *c, uint32_t n_free, jvo_scratch *s,
                        jvo_counts *cnt) {
    for (uint32_t f = 0; f < n_free; ++f) {
        const int32_t start = s->free_rows[f];
        int32_t j = jvo_path(n, c, start, s->y, s->v, s->pred, s->cols, s->d, cnt);
        uint32_t steps = 0;
        int32_t i;
        do {
            i = s->pred[j];
            s->y[j] = i;
            const int32_t prev = s->x[i];
            s->x[i] = j;
            j = prev;
            if (++steps >= n)
                break;
        } while (i != start);
    }
}

/* jonker_internal_flat (jonker_dense_flat.h:260-274) on a square K x K tile.
 * Writes row->col into x_out (int32). */
static void jvo_square(uint32_t n, const float *c, jvo_scratch *s, jvo_counts *cnt) {
    int32_t n_free = jvo_column_reduction(n, c, s, cnt);
    for (int round = 0; n_free > 0 && round < 2; ++round)
        n_free = jvo_row_reduction(n, c, (uint32_t)n_free, s, cnt);
    if (n_free > 0)
        jvo_augment(n, c, (uint32_t)n_free, s, cnt);
}

/* Work model of the device kernel's certified path (not a reference
 * function): the column reduction's claims as the reference's, the transfer
 * taken for every unique row from the column minima at once (each row's
 * minimum over its other columns of c - v, with v the minima before any
 * transfer), then one shortest augmenting path per free row, from the
 * highest free row down, with no augmenting row reduction.  Counted per
 * problem, the searches' scanned rows + paths are the sequential steps that
 * path takes on the device.  Its mapping equals the reference's whenever the
 * optimum is unique (the device keeps it only then). */
static int32_t jvo_column_reduction_parallel(uint32_t n, const float *c, jvo_scratch *s,
                                             jvo_counts *cnt) {
    int32_t *x = s->x, *y = s->y, *fr = s->free_rows;
    float *v = s->v, *v0 = s->d;
    char *unique = s->unique;
    for (uint32_t k = 0; k < n; ++k) {
        unique[k] = 1;
        x[k] = -1;
        v[k] = JVO_LARGE;
        y[k] = 0;
    }
    for (uint32_t i = 0; i < n; ++i) {
        const float *row = c + (size_t)i * n;
        for (uint32_t j = 0; j < n; ++j)
            if (row[j] < v[j]) {
                v[j] = row[j];
                y[j] = (int32_t)i;
            }
    }
    for (int32_t j = (int32_t)n - 1; j >= 0; --j) {
        const int32_t i = y[j];
        if (x[i] < 0) {
            x[i] = j;
        } else {
            unique[i] = 0;
            y[j] = -1;
        }
    }
    for (uint32_t j = 0; j < n; ++j)
        v0[j] = v[j];
    int32_t n_free = 0;
    for (uint32_t i = 0; i < n; ++i) {
        if (x[i] < 0) {
            fr[n_free++] = (int32_t)i;
            continue;
        }
        if (!unique[i])
            continue;
        const int32_t own = x[i];
        const float *row = c + (size_t)i * n;
        float mn = JVO_LARGE;
        for (uint32_t j = 0; j < n; ++j) {
            if ((int32_t)j == own)
                continue;
            const float r = row[j] - v0[j];
            if (r < mn)
                mn = r;
        }
        if (cnt)
            cnt->relax += n - 1;
        v[own] = v0[own] - mn;
    }
    if (cnt)
        cnt->relax += (int64_t)n * n;
    return n_free;
}

static void jvo_sap_square(uint32_t n, const float *c, jvo_scratch *s, jvo_counts *cnt) {
    const int32_t n_free = jvo_column_reduction_parallel(n, c, s, cnt);
    for (int32_t a = 0, b = n_free - 1; a < b; ++a, --b) {
        const int32_t t = s->free_rows[a];
        s->free_rows[a] = s->free_rows[b];
        s->free_rows[b] = t;
    }
    if (n_free > 0)
        jvo_augment(n, c, (uint32_t)n_free, s, cnt);
}

/* ---- jonker_compact_batch: the square JV of jonker_compact_core.h ---------- */

#define JVOC_FLT_MAX 3.402823466e38f /* numeric_limits<float>::max() */

/* find_umins_regular (jonker_compact_core.h:20-43): the smallest reduced
 * cost of row i and the next one in (value, index) order.  Column 0 seeds
 * the minimum; the second minimum starts at FLT_MAX, so an entry that is not
 * below it never becomes j2 (j2 stays -1 when nothing qualifies). */
static void jvoc_two_min(uint32_t n, const float *row, const float *v, float *u1, float *u2,
                         int32_t *j1, int32_t *j2) {
    float lo1 = row[0] - v[0], lo2 = JVOC_FLT_MAX;
    int32_t a = 0, b = -1;
    for (uint32_t j = 1; j < n; ++j) {
        const float h = row[j] - v[j];
        if (!(h < lo2))
            continue;
        if (h >= lo1) {
            lo2 = h;
            b = (int32_t)j;
        } else {
            lo2 = lo1;
            b = a;
            lo1 = h;
            a = (int32_t)j;
        }
    }
    *u1 = lo1;
    *u2 = lo2;
    *j1 = a;
    *j2 = b;
}

/* jonker_compact_kernel<int32_t, float> (jonker_compact_core.h:51-252) on a
 * square n x n tile.  x = rowsol, y = colsol; free_rows doubles as the
 * per-row claim counter of the column reduction, as in the reference
 * (:99).  There is no iteration cap in the reference's augmenting row
 * reduction, and none here. */
static void jvoc_square(uint32_t n, const float *c, jvo_scratch *s, jvo_counts *cnt) {
    int32_t *x = s->x, *y = s->y, *fr = s->free_rows, *pred = s->pred, *cols = s->cols;
    float *v = s->v, *d = s->d;
    int64_t relax = 0, paths = 0, scans = 0;

    /* column reduction, last column first (:73-96): column minimum, first
     * row on ties; the first column (in that order) to reach a row keeps it */
    for (uint32_t i = 0; i < n; ++i)
        fr[i] = 0;
    for (int32_t j = (int32_t)n - 1; j >= 0; --j) {
        float m = c[j];
        int32_t im = 0;
        for (uint32_t i = 1; i < n; ++i)
            if (c[(size_t)i * n + j] < m) {
                m = c[(size_t)i * n + j];
                im = (int32_t)i;
            }
        v[j] = m;
        if (++fr[im] == 1) {
            x[im] = j;
            y[j] = im;
        } else {
            y[j] = -1;
        }
    }
    relax += (int64_t)n * n;

    /* reduction transfer (:98-117): unclaimed rows become free (in row
     * order); a row claimed exactly once lowers its column's dual by its
     * smallest other reduced cost.  fr[] is read at i and written at
     * n_free <= i, so the claim counts are consumed before being overwritten. */
    uint32_t n_free = 0;
    for (uint32_t i = 0; i < n; ++i) {
        const int32_t claims = fr[i];
        if (claims == 0) {
            fr[n_free++] = (int32_t)i;
        } else if (claims == 1) {
            const float *row = c + (size_t)i * n;
            const int32_t jx = x[i];
            float m = JVOC_FLT_MAX;
            for (uint32_t j = 0; j < n; ++j)
                if ((int32_t)j != jx && row[j] - v[j] < m)
                    m = row[j] - v[j];
            v[jx] = v[jx] - m;
            relax += n - 1;
        }
    }

    /* augmenting row reduction, two rounds (:119-166).  A row whose best
     * column's dual can be lowered takes that column and its previous owner
     * is processed next (pushed back at the read position); otherwise it
     * takes the second-best column and the displaced owner waits for the
     * next round (appended at n_free, behind the read position). */
    for (int round = 0; round < 2; ++round) {
        const uint32_t n_prev = n_free;
        uint32_t k = 0;
        n_free = 0;
        while (k < n_prev) {
            const int32_t i = fr[k++];
            float u1, u2;
            int32_t j1, j2;
            jvoc_two_min(n, c + (size_t)i * n, v, &u1, &u2, &j1, &j2);
            relax += n;
            int32_t i0 = y[j1];
            const float lowered = v[j1] - (u2 - u1);
            const int lowers = lowered < v[j1];
            if (lowers) {
                v[j1] = lowered;
            } else if (i0 >= 0) {
                j1 = j2;
                i0 = y[j2];
            }
            x[i] = j1;
            y[j1] = i;
            if (i0 >= 0) {
                if (lowers)
                    fr[--k] = i0;
                else
                    fr[n_free++] = i0;
            }
        }
    }

    /* augmentation (:168-251): one shortest-path search per free row */
    for (uint32_t f = 0; f < n_free; ++f) {
        const int32_t start = fr[f];
        const float *srow = c + (size_t)start * n;
        for (uint32_t j = 0; j < n; ++j) {
            d[j] = srow[j] - v[j];
            pred[j] = start;
            cols[j] = (int32_t)j;
        }
        relax += n;
        ++paths;
        uint32_t low = 0, up = 0;
        int32_t last = 0, end = -1;
        float level = 0.0f;
        while (end < 0) {
            if (up == low) {
                /* gather every column at the new minimum into [low, up):
                 * a smaller d restarts the group at low, an equal one
                 * joins it (:185-199) */
                last = (int32_t)low - 1;
                level = d[cols[up++]];
                for (uint32_t k = up; k < n; ++k) {
                    const int32_t j = cols[k];
                    const float h = d[j];
                    if (h <= level) {
                        if (h < level) {
                            up = low;
                            level = h;
                        }
                        cols[k] = cols[up];
                        cols[up++] = j;
                    }
                }
                /* the first unassigned column of the group ends the path
                 * (:200-206) */
                for (uint32_t k = low; k < up; ++k)
                    if (y[cols[k]] < 0) {
                        end = cols[k];
                        break;
                    }
            }
            if (end >= 0)
                break;
            /* scan the row of the next column of the group (:209-233) */
            const int32_t jq = cols[low++];
            const int32_t iq = y[jq];
            const float *row = c + (size_t)iq * n;
            const float h = row[jq] - v[jq] - level;
            ++scans;
            relax += 1 + (int64_t)(n - up);
            for (uint32_t k = up; k < n; ++k) {
                const int32_t j = cols[k];
                const float r = row[j] - v[j] - h;
                if (!(r < d[j]))
                    continue;
                pred[j] = iq;
                if (r == level) {
                    if (y[j] < 0) {
                        end = j;
                        break;
                    }
                    cols[k] = cols[up];
                    cols[up++] = j;
                }
                d[j] = r;
            }
        }
        /* duals of the columns finished before the last group (:236-239) */
        for (int32_t k = 0; k <= last; ++k) {
            const int32_t j = cols[k];
            v[j] = v[j] + d[j] - level;
        }
        /* flip the assignment along the predecessors (:241-250) */
        int32_t i;
        do {
            i = pred[end];
            y[end] = i;
            const int32_t j = end;
            end = x[i];
            x[i] = j;
        } while (i != start);
    }
    if (cnt) {
        cnt->relax += relax;
        cnt->paths += paths;
        cnt->scans += scans;
    }
}

/* compute_sentinel<float> (ops.cpp:67-93), one serial pass over all cells. */
int jvo_sentinel(const float *data, int64_t count, int32_t K, float *out) {
    float mx = -3.402823466e38f; /* numeric_limits<float>::lowest() */
    int any = 0, nan_seen = 0, neg_inf_seen = 0;
    for (int64_t k = 0; k < count; ++k) {
        const float x = data[k];
        if (isnan(x))
            nan_seen = 1;
        else if (x == -INFINITY)
            neg_inf_seen = 1;
        else if (isfinite(x)) {
            if (x > mx)
                mx = x;
            any = 1;
        }
    }
    if (nan_seen)
        return JVO_ERR_NAN;
    if (neg_inf_seen)
        return JVO_ERR_NEG_INF;
    *out = any ? (mx + 1.0f) * (float)(K + 1) : 1.0f;
    return JVO_OK;
}

/* Pad one problem to K x K: +inf -> sentinel, padding cells 0
 * (ops.cpp:255-270). */
static void jvo_pad(const float *src, int32_t N, int32_t M, int32_t K, float sentinel,
                    float *dst) {
    for (int32_t i = 0; i < K; ++i)
        for (int32_t j = 0; j < K; ++j) {
            float val = 0.0f;
            if (i < N && j < M) {
                val = src[(size_t)i * M + j];
                if (!isfinite(val))
                    val = sentinel;
            }
            dst[(size_t)i * K + j] = val;
        }
}

typedef void (*jvo_solver)(uint32_t, const float *, jvo_scratch *, jvo_counts *);

static int jvo_batch_impl(const float *costs, int64_t B, int32_t N, int32_t M,
                          int64_t *out, int threads, jvo_counts *counts, jvo_solver solve) {
    if (B == 0 || N == 0 || M == 0) {
        for (int64_t k = 0; k < B * (int64_t)N; ++k)
            out[k] = -1;
        return JVO_OK;
    }
    const int32_t K = N > M ? N : M;
    float sentinel = 1.0f;
    const int rc = jvo_sentinel(costs, B * (int64_t)N * M, K, &sentinel);
    if (rc != JVO_OK)
        return rc;
    int failed = 0;
#ifdef _OPENMP
    if (threads <= 0)
        threads = omp_get_max_threads();
#pragma omp parallel num_threads(threads) reduction(| : failed)
#endif
    {
        float *tile = (float *)malloc(sizeof(float) * (size_t)K * K);
        int32_t *ibuf = (int32_t *)malloc(sizeof(int32_t) * (size_t)K * 5);
        float *fbuf = (float *)malloc(sizeof(float) * (size_t)K * 2);
        char *ubuf = (char *)malloc((size_t)K);
        if (!tile || !ibuf || !fbuf || !ubuf) {
            failed = 1;
        } else {
            jvo_scratch s = {ibuf, ibuf + K, ibuf + 2 * K, ibuf + 3 * K, ibuf + 4 * K,
                             fbuf, fbuf + K, ubuf};
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
            for (int64_t b = 0; b < B; ++b) {
                jvo_pad(costs + b * (int64_t)N * M, N, M, K, sentinel, tile);
                solve((uint32_t)K, tile, &s, counts ? &counts[b] : NULL);
                for (int32_t i = 0; i < N; ++i) {
                    const int32_t j = s.x[i];
                    out[b * N + i] = (j >= 0 && j < M) ? j : -1;
                }
            }
        }
        free(tile);
        free(ibuf);
        free(fbuf);
        free(ubuf);
    }
    (void)threads;
    return failed ? JVO_ERR_ALLOC : JVO_OK;
}

/* Public entry: (B, N, M) float32 contiguous -> (B, N) int64.
 * threads <= 0 means "all OpenMP threads".  Returns 0, or 1 (NaN), 2 (-inf),
 * 3 (allocation failure). */
int jvo_dense_batch(const float *costs, int64_t B, int32_t N, int32_t M, int64_t *out,
                    int threads) {
    return jvo_batch_impl(costs, B, N, M, out, threads, NULL, jvo_square);
}

/* jonker_compact_batch: the same batch driver (ops.cpp:431-433 runs
 * solve_batch with the compact solver) around jvoc_square. */
int jvo_compact_batch(const float *costs, int64_t B, int32_t N, int32_t M, int64_t *out,
                      int threads) {
    return jvo_batch_impl(costs, B, N, M, out, threads, NULL, jvoc_square);
}

/* Same, single-threaded, with per-problem work counters (3 int64 per problem:
 * relaxations, paths, scanned rows). */
int jvo_dense_batch_counted(const float *costs, int64_t B, int32_t N, int32_t M,
                            int64_t *out, int64_t *counts3) {
    jvo_counts *cnt = (jvo_counts *)calloc((size_t)(B > 0 ? B : 1), sizeof(jvo_counts));
    if (!cnt)
        return JVO_ERR_ALLOC;
    const int rc = jvo_batch_impl(costs, B, N, M, out, 1, cnt, jvo_square);
    for (int64_t b = 0; b < B; ++b) {
        counts3[3 * b + 0] = cnt[b].relax;
        counts3[3 * b + 1] = cnt[b].paths;
        counts3[3 * b + 2] = cnt[b].scans;
    }
    free(cnt);
    return rc;
}

/* The reference order's sequential steps per problem, single-threaded (3 int64
 * per problem: augmenting row reduction steps, paths, rows scanned in the
 * paths' searches).  A solver that follows the reference's order takes these
 * steps one after another; their total on the slowest problem bounds a
 * launch from below. */
int jvo_dense_batch_steps(const float *costs, int64_t B, int32_t N, int32_t M, int64_t *out,
                          int64_t *steps3) {
    jvo_counts *cnt = (jvo_counts *)calloc((size_t)(B > 0 ? B : 1), sizeof(jvo_counts));
    if (!cnt)
        return JVO_ERR_ALLOC;
    const int rc = jvo_batch_impl(costs, B, N, M, out, 1, cnt, jvo_square);
    for (int64_t b = 0; b < B; ++b) {
        steps3[3 * b + 0] = cnt[b].rr_steps;
        steps3[3 * b + 1] = cnt[b].paths;
        steps3[3 * b + 2] = cnt[b].scans;
    }
    free(cnt);
    return rc;
}

/* jvo_sap_square over a batch, single-threaded, with the same counters. */
int jvo_sap_batch_counted(const float *costs, int64_t B, int32_t N, int32_t M, int64_t *out,
                          int64_t *counts3) {
    jvo_counts *cnt = (jvo_counts *)calloc((size_t)(B > 0 ? B : 1), sizeof(jvo_counts));
    if (!cnt)
        return JVO_ERR_ALLOC;
    const int rc = jvo_batch_impl(costs, B, N, M, out, 1, cnt, jvo_sap_square);
    for (int64_t b = 0; b < B; ++b) {
        counts3[3 * b + 0] = cnt[b].relax;
        counts3[3 * b + 1] = cnt[b].paths;
        counts3[3 * b + 2] = cnt[b].scans;
    }
    free(cnt);
    return rc;
}
