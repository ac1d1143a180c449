// planner.cpp -- host planning of the row kernel's wavefront task list and
// the condensed-window indexing.
#include "planner.hpp"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <numeric>

#include <omp.h>

#include "common.hpp"

namespace tca {

namespace {
constexpr int kUnroll = 8;  // loads in flight per lane in the row kernel

int32_t next_pow2(int64_t x) {
    int32_t p = 1;
    while (p < x) p <<= 1;
    return p;
}
int32_t ilog2(int32_t x) {
    int32_t l = 0;
    while ((1 << l) < x) l++;
    return l;
}
}  // namespace

int32_t default_slices(int32_t K, int32_t N, int32_t dtype) {
    if (const char* sl = std::getenv("TCA_SLICES")) return std::atoi(sl);
    const uint64_t b_bytes = static_cast<uint64_t>(K) * static_cast<uint64_t>(N) * dtype_size(dtype);
    return b_bytes > (8ull << 20) ? 0 : 1;
}

void plan_geometry(int32_t N, int32_t es, int32_t slices, RowPlan* p) {
    int32_t e = 16 / es;
    while (e > 1 && N % e != 0) e >>= 1;
    p->elems_per_lane = e;
    const int64_t lanes = N / e;  // 16-byte (or narrower) vectors across one B row
    int64_t nch = 1;
    if (slices > 0) {
        nch = slices;
    } else {
        // Up to 8 chunks (one per XCD), each at least one 128-byte L2 line wide.
        while (nch < 8 && lanes % (2 * nch) == 0 && (lanes / (2 * nch)) * e * es >= 128) nch *= 2;
    }
    while ((lanes + nch - 1) / nch > 64) nch *= 2;  // at most 64 lanes per chunk
    p->col_chunks = static_cast<int32_t>(nch);
    p->chunk_lanes = static_cast<int32_t>((lanes + nch - 1) / nch);
    p->log_lanes = ilog2(next_pow2(p->chunk_lanes));
}

void plan_row_params(int64_t nnz, int32_t N, int32_t es, int32_t slices, RowPlan* p) {
    plan_geometry(N, es, slices, p);
    const int32_t slots = 64 >> p->log_lanes;
    // Work per wavefront task: about nnz / 32768 nonzeros (four resident
    // wavefronts on each of 256 CUs x 4 SIMDs x 8 slots, so long rows do
    // not leave a latency tail), a power of two of at least 256 nonzeros and
    // 2 rounds of slots * kUnroll loads, at most 32 rounds.  (Shorter tasks
    // cost more in partial sums than they gain in balance: on MI355X the
    // 4096 x 4096 config-1 matrix runs 44 us at 256 and 47 us at 64;
    // config 4, 20M nonzeros mostly in long rows' segments: 251 us at 2048,
    // 212 at 1024, 217 at 512, 250 at 256.)
    const int64_t round = static_cast<int64_t>(slots) * kUnroll;
    int64_t target = next_pow2(std::max<int64_t>(nnz / 32768, 1));
    target = std::min<int64_t>(std::max<int64_t>(32 * round, 256), std::max<int64_t>({2 * round, 256, target}));
    // Tuning overrides (not part of the interface): TCA_TARGET sets the
    // per-task length, TCA_WIDE=0 disables workgroup-shared rows,
    // TCA_MULTI sets the multi-task row-length limit.
    if (const char* s = std::getenv("TCA_TARGET")) target = std::max<int64_t>(round, std::atoll(s));
    p->row_len = static_cast<int32_t>(target);
    const char* w = std::getenv("TCA_WIDE");
    p->wide_len = static_cast<int32_t>((w && std::atoi(w) == 0) ? target : 4 * target);
    p->seg_len = static_cast<int32_t>(target);
    // Short rows share a wavefront, one slot each, when slots > 1.
    p->multi_max = slots > 1 ? 2 * slots : -1;
    if (const char* s = std::getenv("TCA_MULTI")) p->multi_max = slots > 1 ? std::atoi(s) : -1;
}

void plan_rows(const int32_t* rowptr, int32_t M, int32_t N, int32_t es, const std::vector<uint8_t>& skip,
               int32_t slices, RowPlan* p) {
    plan_row_params(rowptr[M], N, es, slices, p);
    const int32_t slots = 64 >> p->log_lanes;

    std::vector<int32_t> rows;
    rows.reserve(M);
    for (int32_t r = 0; r < M; r++)
        if (skip.empty() || !skip[r]) rows.push_back(r);
    auto len = [&](int32_t r) { return rowptr[r + 1] - rowptr[r]; };
    // Longest first; row id breaks ties so the plan is deterministic.
    std::stable_sort(rows.begin(), rows.end(), [&](int32_t a, int32_t b) { return len(a) > len(b); });

    p->tasks.clear();
    p->perm.clear();
    p->longrows.clear();
    size_t i = 0;
    while (i < rows.size() && len(rows[i]) > p->wide_len) i++;
    const size_t n_long = i;
    // Wide rows: four quarters, one per wavefront of a workgroup (4-aligned).
    for (; i < rows.size() && len(rows[i]) > p->row_len; i++) {
        const int32_t r = rows[i];
        const int64_t L = len(r);
        for (int32_t q = 0; q < 4; q++)
            p->tasks.push_back({r, rowptr[r] + static_cast<int32_t>(L * q / 4),
                                rowptr[r] + static_cast<int32_t>(L * (q + 1) / 4), kTaskWide | (q << 2)});
    }
    p->n_wide = static_cast<int32_t>(p->tasks.size());
    const size_t first_row = i;
    // Long rows: equal segments of at most seg_len nonzeros, summed by a second kernel.
    int32_t seg_global = 0;
    for (size_t k = 0; k < n_long; k++) {
        const int32_t r = rows[k];
        const int32_t L = len(r);
        const int32_t nseg = (L + p->seg_len - 1) / p->seg_len;
        const int32_t lid = static_cast<int32_t>(p->longrows.size());
        p->longrows.push_back({r, seg_global, nseg, 0});
        for (int32_t s = 0; s < nseg; s++) {
            const int32_t b = rowptr[r] + static_cast<int32_t>(static_cast<int64_t>(L) * s / nseg);
            const int32_t e = rowptr[r] + static_cast<int32_t>(static_cast<int64_t>(L) * (s + 1) / nseg);
            p->tasks.push_back({lid, b, e, kTaskSeg | ((seg_global + s) << 2)});
        }
        seg_global += nseg;
    }
    p->n_seg = static_cast<int32_t>(p->tasks.size()) - p->n_wide;
    // Medium rows: one wavefront each.
    for (i = first_row; i < rows.size() && len(rows[i]) > std::max(p->multi_max, 0); i++) {
        const int32_t r = rows[i];
        p->tasks.push_back({r, rowptr[r], rowptr[r + 1], kTaskRow});
    }
    p->n_rowtasks = static_cast<int32_t>(p->tasks.size()) - p->n_seg - p->n_wide;
    // Short rows: groups of multi_group_rows(slots) rows of similar length;
    // empty rows (the tail of the order) in groups of kZeroRows, which only
    // clear their C rows.
    const size_t first_multi = p->tasks.size();
    size_t end_nz = i;
    while (end_nz < rows.size() && len(rows[end_nz]) > 0) end_nz++;
    for (size_t k = i; k < rows.size();) {
        const size_t lim = k < end_nz ? std::min<size_t>(k + multi_group_rows(slots), end_nz)
                                      : std::min<size_t>(k + kZeroRows, rows.size());
        p->tasks.push_back({static_cast<int32_t>(p->perm.size()), static_cast<int32_t>(lim - k), len(rows[k]), kTaskMulti});
        for (; k < lim; k++) p->perm.push_back(rows[k]);
    }
    p->n_multi = static_cast<int32_t>(p->tasks.size() - first_multi);
}

void condense(const int32_t* rowptr, const int32_t* colidx, int32_t M, int32_t win, std::vector<int64_t>* uoff,
              std::vector<int32_t>* ucols, std::vector<int32_t>* cpos) {
    const int32_t nw = (M + win - 1) / win;
    uoff->assign(static_cast<size_t>(nw) + 1, 0);
    std::vector<std::vector<int32_t>> u(nw);
#pragma omp parallel for schedule(dynamic, 16)
    for (int32_t w = 0; w < nw; w++) {
        const int32_t s = rowptr[static_cast<int64_t>(w) * win];
        const int32_t e = rowptr[std::min<int64_t>(M, static_cast<int64_t>(w + 1) * win)];
        std::vector<int32_t>& uw = u[w];
        uw.assign(colidx + s, colidx + e);
        std::sort(uw.begin(), uw.end());
        uw.erase(std::unique(uw.begin(), uw.end()), uw.end());
        if (cpos)
            for (int32_t j = s; j < e; j++)
                (*cpos)[j] = static_cast<int32_t>(std::lower_bound(uw.begin(), uw.end(), colidx[j]) - uw.begin());
    }
    for (int32_t w = 0; w < nw; w++) (*uoff)[w + 1] = (*uoff)[w] + static_cast<int64_t>(u[w].size());
    if (ucols) {
        ucols->resize((*uoff)[nw]);
        for (int32_t w = 0; w < nw; w++) std::copy(u[w].begin(), u[w].end(), ucols->begin() + (*uoff)[w]);
    }
}

void route_windows(const std::vector<WinStat>& st, int32_t M, int64_t nnz_total, int32_t N, bool force,
                   double min_density, const MfmaShape& shape, std::vector<uint8_t>* take_out) {
    constexpr int32_t kStep = 32;
    const int32_t kWin = shape.win_rows, kMaxStep = shape.max_step_entries;
    const int32_t nw = static_cast<int32_t>(st.size());
    std::vector<uint8_t>& take = *take_out;
    take.assign(nw, 0);
    std::vector<uint8_t> ok(nw, 0);  // structurally able
    for (int32_t w = 0; w < nw; w++) {
        const int32_t r0 = w * kWin, r1 = std::min(M, r0 + kWin);
        const int64_t nz = st[w].nz;
        if (nz == 0 || nz >= (int64_t(1) << 20)) continue;
        const int64_t steps = (st[w].ucount + kStep - 1) / kStep;
        // nonzeros per step must fit the kernel's entry slots
        if (st[w].maxper > kMaxStep) continue;
        const double density = static_cast<double>(nz) / (static_cast<double>(r1 - r0) * steps * kStep);
        ok[w] = 1;
        if (force || density >= min_density) take[w] = 1;
    }
    if (!force) {
        // Cost model over the eligible set (see planner.hpp).
        int64_t n_take = 0, nz_take = 0, max_steps = 0;
        for (int32_t w = 0; w < nw; w++) {
            if (!take[w]) continue;
            n_take++;
            nz_take += st[w].nz;
            max_steps = std::max<int64_t>(max_steps, (st[w].ucount + kStep - 1) / kStep);
        }
        const int64_t wgs = n_take * ((N + shape.tile_cols - 1) / shape.tile_cols);
        const int64_t rounds = (wgs + 255) / 256;
        const double t_tile =
            shape.fixed_us + static_cast<double>(rounds) * ((max_steps + 3) / 4 + shape.fill_iters) * shape.iter_us;
        const double t_row = static_cast<double>(nz_take) * N * 2.0 / kRowGatherBytesPerUs;
        if (n_take > 0 && t_tile >= t_row) {
            std::fill(take.begin(), take.end(), 0);
        } else if (n_take > 0 && static_cast<double>(nz_take) >= 0.95 * nnz_total) {
            // Nearly everything goes to the tile kernel: take the remaining
            // qualifying windows too rather than launch the row kernel for a
            // few rows (the launch alone costs more than their tiles).
            std::copy(ok.begin(), ok.end(), take.begin());
        }
    }
}

void plan_mfma(const int32_t* rowptr, const int32_t* colidx, int32_t M, int32_t N, int32_t dtype, bool force,
               bool disable, double min_density, const MfmaShape& shape, MfmaPlan* p) {
    constexpr int32_t kStep = 32;
    const int32_t kWin = shape.win_rows;
    *p = MfmaPlan();
    p->win_rows = kWin;
    p->row_mfma.assign(M, 0);
    if (disable || dtype == TCA_F32 || N % 8 != 0 || M == 0) return;
    std::vector<int64_t> uoff;
    std::vector<int32_t> ucols, cpos(rowptr[M]);
    condense(rowptr, colidx, M, kWin, &uoff, &ucols, &cpos);
    const int32_t nw = (M + kWin - 1) / kWin;
    std::vector<WinStat> st(nw);
#pragma omp parallel for schedule(dynamic, 16)
    for (int32_t w = 0; w < nw; w++) {
        const int32_t r0 = w * kWin, r1 = std::min(M, r0 + kWin);
        st[w].nz = rowptr[r1] - rowptr[r0];
        st[w].ucount = static_cast<int32_t>(uoff[w + 1] - uoff[w]);
        st[w].maxper = 0;
        if (st[w].nz == 0) continue;
        const int64_t steps = (st[w].ucount + kStep - 1) / kStep;
        std::vector<int32_t> per(steps, 0);
        for (int32_t j = rowptr[r0]; j < rowptr[r1]; j++) per[cpos[j] / kStep]++;
        st[w].maxper = *std::max_element(per.begin(), per.end());
    }
    std::vector<uint8_t> take;
    route_windows(st, M, rowptr[M], N, force, min_density, shape, &take);
    for (int32_t w = 0; w < nw; w++) {
        if (!take[w]) continue;
        const int32_t r0 = w * kWin, r1 = std::min(M, r0 + kWin);
        const int32_t ucount = static_cast<int32_t>(uoff[w + 1] - uoff[w]);
        const int32_t steps = (ucount + kStep - 1) / kStep;
        const int32_t gstep = static_cast<int32_t>(p->eoff.size());
        p->windows.push_back({r0, steps, gstep, rowptr[r0]});
        for (int32_t s = 0; s < steps * kStep; s++)
            p->ucols.push_back(s < ucount ? ucols[uoff[w] + s] : -1);
        // entries bucketed by step; rows in order and columns ascending inside
        // a row, so each bucket lists (row, column) in row-major order
        std::vector<int32_t> cnt(steps + 1, 0);
        for (int32_t j = rowptr[r0]; j < rowptr[r1]; j++) cnt[cpos[j] / kStep + 1]++;
        for (int32_t s = 0; s < steps; s++) cnt[s + 1] += cnt[s];
        const size_t ebase = p->entries.size();
        for (int32_t s = 0; s < steps; s++) p->eoff.push_back(static_cast<int32_t>(ebase + cnt[s]));
        p->entries.resize(ebase + cnt[steps]);
        std::vector<int32_t> fill(cnt.begin(), cnt.end() - 1);
        for (int32_t r = r0; r < r1; r++)
            for (int32_t j = rowptr[r]; j < rowptr[r + 1]; j++) {
                const int32_t s = cpos[j] / kStep;
                p->entries[ebase + fill[s]++] = static_cast<uint32_t>(r - r0) |
                                                (static_cast<uint32_t>(cpos[j] % kStep) << 7) |
                                                (static_cast<uint32_t>(j - rowptr[r0]) << 12);
            }
        for (int32_t r = r0; r < r1; r++) p->row_mfma[r] = 1;
        p->nnz += rowptr[r1] - rowptr[r0];
        p->cond_cols += static_cast<int64_t>(steps) * kStep;
        p->rows += r1 - r0;
    }
    p->eoff.push_back(static_cast<int32_t>(p->entries.size()));
}

int32_t panel_elems(int32_t N, int32_t es) {
    for (int32_t e = 8; e >= 2; e >>= 1)
        if (N % (16 * e) == 0 && e * es >= 8 && e * es <= 32) return e;
    return 0;
}

bool panel_default_ok(int32_t N, int32_t es) {
    // B rows of at least 256 bytes: with narrower rows the row kernel's
    // gathers are cheap and win (measured on MI355X, configuration 4, fp16
    // N = 64: 0.60 ms with panels, 0.44 ms on the row kernel alone).
    const int32_t e = panel_elems(N, es);
    return e > 0 && static_cast<int64_t>(N) * es >= 256;
}

int32_t panel_tile_cols(int32_t chunk_bytes) { return std::min<int32_t>(255, 77824 / chunk_bytes); }

bool panel_route(int32_t K, int32_t N, int32_t dtype, uint32_t flags, PanelRoute* r) {
    *r = PanelRoute{};
    if ((flags & TCA_PLAN_NO_PANELS) ||
        (!(flags & TCA_PLAN_FORCE_PANELS) && !panel_default_ok(N, static_cast<int32_t>(dtype_size(dtype)))))
        return false;
    r->force = (flags & TCA_PLAN_FORCE_PANELS) != 0;
    // With B past the MALL the row kernel's per-nonzero gathers come from
    // HBM, and even rows that share no columns cost less staged (measured
    // on MI355X, config 3, B 1.25 GB: every row with nonzeros in panels
    // 2.564-2.573 ms against 2.600-2.608 at reuse 1.02, one box; config 2,
    // B 119 MB: 1.66-1.72 against 1.54-1.57 ms).
    const bool b_past_mall = static_cast<int64_t>(K) * N * static_cast<int64_t>(dtype_size(dtype)) > kMallBytes;
    r->min_reuse = b_past_mall ? 0.0 : kPanelMinReuse;
    r->min_nnz = kPanelMinNnz;
    r->unit_nnz = 0;
    // Tuning overrides (not part of the interface).
    if (const char* e = std::getenv("TCA_PANEL_MIN_REUSE")) r->min_reuse = std::atof(e);
    if (const char* e = std::getenv("TCA_PANEL_MIN_NNZ")) r->min_nnz = std::atoll(e);
    if (const char* e = std::getenv("TCA_PANEL_UNIT")) r->unit_nnz = std::atoll(e);
    return true;
}

int64_t panel_unit_nnz(int64_t unit_nnz, int64_t tot) {
    // Units of ~1/320 of the panels' nonzeros: about one per CU, so each CU
    // works through one contiguous column range of a panel and the partial
    // rows stay few (measured on MI355X, per SpMM, config 2 / config 3:
    // tot / 2048 1.87 / 3.34 ms, / 1024 1.69 / 3.23, / 512 1.65 / 3.24,
    // / 256 1.63 / 3.07, / 128 - / 3.67, one box; then on another, config 3:
    // / 256 3.15, / 320 3.03-3.04, / 192 3.08-3.13, config 2 level within
    // the box's 5 % noise).
    return unit_nnz > 0 ? unit_nnz : std::max<int64_t>(8192, tot / 320);
}

void plan_panels_routed(const int32_t* rowptr, const int32_t* colidx, int32_t M, int32_t K, int32_t N,
                        int32_t dtype, uint32_t flags, const std::vector<uint8_t>& skip, PanelPlan* p) {
    PanelRoute r;
    if (!panel_route(K, N, dtype, flags, &r)) {
        *p = PanelPlan{};
        p->row_panel.assign(M, 0);
        return;
    }
    plan_panels(rowptr, colidx, M, K, N, static_cast<int32_t>(dtype_size(dtype)), skip, r.force, r.min_reuse,
                r.min_nnz, r.unit_nnz, p);
}

void plan_panels(const int32_t* rowptr, const int32_t* colidx, int32_t M, int32_t K, int32_t N, int32_t es,
                 const std::vector<uint8_t>& skip, bool force, double min_reuse, int64_t min_nnz, int64_t unit_nnz,
                 PanelPlan* p) {
    *p = PanelPlan{};
    p->row_panel.assign(M, 0);
    const int32_t E = panel_elems(N, es);
    if (E == 0 || M == 0) return;
    p->elems = E;
    p->chunks = N / (16 * E);
    p->waves = kPanelWaves;
    p->rpg = kPanelRpg;
    p->R = p->waves * 4 * p->rpg;
    p->P = panel_tile_cols(16 * E * es);
    const int32_t R = p->R, P = p->P, G = p->waves * 4;
    auto len = [&](int32_t r) { return rowptr[r + 1] - rowptr[r]; };

    std::vector<int32_t> order;
    order.reserve(M);
    for (int32_t r = 0; r < M; r++)
        if ((skip.empty() || !skip[r]) && len(r) > 0) order.push_back(r);
    std::stable_sort(order.begin(), order.end(), [&](int32_t a, int32_t b) { return len(a) > len(b); });
    const int32_t n_cand = static_cast<int32_t>((order.size() + R - 1) / R);
    if (n_cand == 0) return;

    // Pass 1 (parallel over candidate panels): slot assignment, sorted column
    // union, and whether the panel is taken.
    struct Cand {
        std::vector<int32_t> slots;  // R entries: row id or -1
        std::vector<int32_t> uni;
        std::vector<int32_t> cuts;  // tile t = union positions [cuts[t], cuts[t + 1])
        int64_t nnz = 0;
        bool take = false;
    };
    std::vector<Cand> cand(n_cand);
#pragma omp parallel
    {
        std::vector<int32_t> mark(K, -1), posmap(K, 0);
#pragma omp for schedule(dynamic, 1)
        for (int32_t q = 0; q < n_cand; q++) {
            Cand& c = cand[q];
            c.slots.assign(R, -1);
            const size_t first = static_cast<size_t>(q) * R;
            const size_t cnt = std::min<size_t>(R, order.size() - first);
            for (size_t k = 0; k < cnt; k++) {
                // k-th longest row of the panel -> group k % G, row entry k / G
                const int32_t gi = static_cast<int32_t>(k % G), i = static_cast<int32_t>(k / G);
                const int32_t wave = gi / 4, group = gi % 4;
                const int32_t row = order[first + k];
                c.slots[(wave * p->rpg + i) * 4 + group] = row;
                c.nnz += len(row);
                for (int32_t j = rowptr[row]; j < rowptr[row + 1]; j++)
                    if (mark[colidx[j]] != q) {
                        mark[colidx[j]] = q;
                        c.uni.push_back(colidx[j]);
                    }
            }
            std::sort(c.uni.begin(), c.uni.end());
            c.take = !c.uni.empty() && (force || static_cast<double>(c.nnz) >= min_reuse * c.uni.size());
            if (!c.take) {
                c.uni.clear();
                continue;
            }
            // Tiles: ranges of the union of at most P columns in which no row
            // holds more than kPanelMaxRun nonzeros (one 16-lane batch).
            const int32_t U = static_cast<int32_t>(c.uni.size());
            for (int32_t u = 0; u < U; u++) posmap[c.uni[u]] = u;
            std::vector<int32_t> head(U + 1, 0);  // slots holding union column u: colslot[head[u] .. head[u+1])
            for (int32_t s = 0; s < R; s++) {
                const int32_t row = c.slots[s];
                if (row >= 0)
                    for (int32_t j = rowptr[row]; j < rowptr[row + 1]; j++) head[posmap[colidx[j]] + 1]++;
            }
            for (int32_t u = 0; u < U; u++) head[u + 1] += head[u];
            std::vector<uint16_t> colslot(head[U]);
            {
                std::vector<int32_t> fill(head.begin(), head.end() - 1);
                for (int32_t s = 0; s < R; s++) {
                    const int32_t row = c.slots[s];
                    if (row >= 0)
                        for (int32_t j = rowptr[row]; j < rowptr[row + 1]; j++)
                            colslot[fill[posmap[colidx[j]]]++] = static_cast<uint16_t>(s);
                }
            }
            std::vector<int32_t> run(R, 0);
            c.cuts.assign(1, 0);
            for (int32_t u = 0; u < U; u++) {
                bool cut = u - c.cuts.back() == P;
                for (int32_t h = head[u]; h < head[u + 1] && !cut; h++) cut = run[colslot[h]] == kPanelMaxRun;
                if (cut) {
                    for (int32_t v = c.cuts.back(); v < u; v++)
                        for (int32_t h = head[v]; h < head[v + 1]; h++) run[colslot[h]] = 0;
                    c.cuts.push_back(u);
                }
                for (int32_t h = head[u]; h < head[u + 1]; h++) run[colslot[h]]++;
            }
            c.cuts.push_back(U);
        }
    }

    // Tile and unit layout (sequential: global offsets).
    int64_t tot = 0;
    for (const Cand& c : cand)
        if (c.take) tot += c.nnz;
    // Too few nonzeros for the panel kernel's workgroups to fill the GPU: the
    // row kernel's short tasks do better (measured on the 2048 x 512
    // configuration 0, 105k nonzeros: 52.6 us on panels, 5.6 us on rows).
    if (tot == 0 || (!force && tot < min_nnz)) {
        p->n_panels = 0;
        p->rows.clear();
        p->cols.clear();
        p->width.clear();
        p->cnt.clear();
        p->pos.clear();
        return;
    }
    unit_nnz = panel_unit_nnz(unit_nnz, tot);
    std::vector<int32_t> panel_of(n_cand, -1), tile0(n_cand, 0);
    int32_t n_tiles = 0;
    for (int32_t q = 0; q < n_cand; q++) {
        if (!cand[q].take) continue;
        panel_of[q] = p->n_panels++;
        tile0[q] = n_tiles;
        n_tiles += static_cast<int32_t>(cand[q].cuts.size()) - 1;
    }
    p->rows.assign(static_cast<size_t>(p->n_panels) * R, -1);
    p->cols.assign(static_cast<size_t>(n_tiles) * P, 0);
    p->width.assign(n_tiles, 0);
    const size_t cnt_stride = static_cast<size_t>(p->waves) * kPanelCntRows * 4;  // bytes per tile
    p->cnt.assign(static_cast<size_t>(n_tiles) * cnt_stride, 0);
    p->pos.assign((static_cast<size_t>(rowptr[M]) + 3) & ~size_t(3), 0);  // whole dwords (the kernel loads dwords)

    // Pass 2 (parallel over taken panels): positions, counts.
#pragma omp parallel
    {
        std::vector<int32_t> posmap(K, 0);
#pragma omp for schedule(dynamic, 1)
        for (int32_t q = 0; q < n_cand; q++) {
            if (!cand[q].take) continue;
            const Cand& c = cand[q];
            const int32_t pid = panel_of[q], t0 = tile0[q];
            const int32_t U = static_cast<int32_t>(c.uni.size());
            const int32_t nt = static_cast<int32_t>(c.cuts.size()) - 1;
            std::vector<int32_t> tile_of(U);
            for (int32_t t = 0; t < nt; t++) {
                p->width[t0 + t] = static_cast<uint8_t>(c.cuts[t + 1] - c.cuts[t]);
                for (int32_t u = c.cuts[t]; u < c.cuts[t + 1]; u++) tile_of[u] = t;
                for (int32_t j = 0; j < P; j++)  // padding repeats the tile's last column
                    p->cols[static_cast<size_t>(t0 + t) * P + j] = c.uni[std::min(c.cuts[t] + j, c.cuts[t + 1] - 1)];
            }
            for (int32_t u = 0; u < U; u++) posmap[c.uni[u]] = u;
            for (int32_t s = 0; s < R; s++) {
                const int32_t row = c.slots[s];
                p->rows[static_cast<size_t>(pid) * R + s] = row;
                if (row < 0) continue;
                const int32_t wave = s / (4 * p->rpg), i = (s / 4) % p->rpg, group = s % 4;
                for (int32_t k = rowptr[row]; k < rowptr[row + 1]; k++) {
                    const int32_t u = posmap[colidx[k]];
                    const int32_t t = tile_of[u];
                    p->pos[k] = static_cast<uint8_t>(u - c.cuts[t] + 1);
                    p->cnt[static_cast<size_t>(t0 + t) * cnt_stride + (wave * kPanelCntRows + i) * 4 + group]++;
                }
                p->row_panel[row] = 1;
            }
            // per wave and entry: the longest of the four group counts
            for (int32_t t = 0; t < nt; t++) {
                uint8_t* cb = &p->cnt[static_cast<size_t>(t0 + t) * cnt_stride];
                for (int32_t wave = 0; wave < p->waves; wave++)
                    for (int32_t i = 0; i < p->rpg; i++) {
                        const uint8_t* c4 = cb + (wave * kPanelCntRows + i) * 4;
                        cb[(wave * kPanelCntRows + kPanelMaxDword + i / 4) * 4 + i % 4] =
                            std::max(std::max(c4[0], c4[1]), std::max(c4[2], c4[3]));
                    }
            }
        }
    }

    // Units: each panel's tiles, split by nonzeros into units of ~unit_nnz.
    int64_t seg = 0;
    for (int32_t q = 0; q < n_cand; q++) {
        if (!cand[q].take) continue;
        const Cand& c = cand[q];
        const int32_t pid = panel_of[q], t0 = tile0[q];
        const int32_t nt = static_cast<int32_t>(c.cuts.size()) - 1;
        const int32_t nu = static_cast<int32_t>(std::max<int64_t>(1, std::min<int64_t>(nt, (c.nnz + unit_nnz - 1) / unit_nnz)));
        // tile nonzeros, then cut points at multiples of nnz / nu
        std::vector<int64_t> tn(nt, 0);
        for (int32_t t = 0; t < nt; t++) {
            const uint8_t* cb = &p->cnt[static_cast<size_t>(t0 + t) * cnt_stride];
            for (int32_t wave = 0; wave < p->waves; wave++)
                for (int32_t b = 0; b < p->rpg * 4; b++) tn[t] += cb[wave * kPanelCntRows * 4 + b];
        }
        std::vector<int32_t> cut = {0};
        int64_t acc = 0;
        for (int32_t t = 0; t < nt; t++) {
            acc += tn[t];
            const int64_t want = c.nnz * static_cast<int64_t>(cut.size()) / nu;
            if (acc >= want && static_cast<int32_t>(cut.size()) < nu && t + 1 < nt) cut.push_back(t + 1);
        }
        cut.push_back(nt);
        const int32_t units = static_cast<int32_t>(cut.size()) - 1;
        const int32_t first_seg = units > 1 ? static_cast<int32_t>(seg) : -1;
        // per slot cursor walking the tiles
        std::vector<int32_t> cur(R, 0);
        for (int32_t s = 0; s < R; s++) cur[s] = c.slots[s] >= 0 ? rowptr[c.slots[s]] : 0;
        for (int32_t k = 0; k < units; k++) {
            p->units.push_back({pid, t0 + cut[k], cut[k + 1] - cut[k], units > 1 ? first_seg + k : -1});
            for (int32_t s = 0; s < R; s++) p->ustart.push_back(cur[s]);
            for (int32_t t = cut[k]; t < cut[k + 1]; t++) {
                const uint8_t* cb = &p->cnt[static_cast<size_t>(t0 + t) * cnt_stride];
                for (int32_t s = 0; s < R; s++) {
                    const int32_t wave = s / (4 * p->rpg), i = (s / 4) % p->rpg, group = s % 4;
                    cur[s] += cb[(wave * kPanelCntRows + i) * 4 + group];
                }
            }
        }
        p->panel_units.push_back(units);
        if (units > 1) {
            for (int32_t s = 0; s < R; s++)
                if (c.slots[s] >= 0) p->longrows.push_back({c.slots[s], first_seg + s * units, units, 0});
            seg += static_cast<int64_t>(R) * units;
        }
        p->nnz += c.nnz;
        p->staged += static_cast<int64_t>(c.uni.size());
        p->win.push_back(panel_window(c.nnz, static_cast<int64_t>(c.uni.size())) ? 1 : 0);
        for (int32_t s = 0; s < R; s++) p->n_rows += c.slots[s] >= 0;
    }
    p->n_segments = seg;
    order_units(K, p);
}

bool panel_window(int64_t nnz, int64_t staged) {
    if (const char* e = std::getenv("TCA_PANEL_WINDOW")) return std::atoi(e) != 0;
    double reuse = kPanelWindowReuse;
    if (const char* e = std::getenv("TCA_PANEL_WINDOW_REUSE")) reuse = std::atof(e);  // tuning override
    return static_cast<double>(nnz) < reuse * static_cast<double>(staged);
}

void order_units(int32_t K, PanelPlan* p) {
    const size_t nu = p->units.size();
    std::vector<int64_t> lo(nu), hi(nu);
    for (size_t u = 0; u < nu; u++) {
        const Int4& t = p->units[u];
        lo[u] = p->cols[static_cast<size_t>(t.y) * p->P];
        hi[u] = p->cols[static_cast<size_t>(t.y + t.z) * p->P - 1];  // padding repeats the last column
    }
    order_unit_spans(K, p->chunks, p->units, lo, hi, &p->order);
}

void order_unit_spans(int32_t K, int32_t chunks, const std::vector<Int4>& units, const std::vector<int64_t>& lo,
                      const std::vector<int64_t>& hi, std::vector<int32_t>* order) {
    const int32_t nu = static_cast<int32_t>(units.size());
    order->clear();
    const char* e = std::getenv("TCA_PANEL_ORDER");  // tuning override: 0 = natural order
    if (chunks != 1 || (e && std::atoi(e) == 0)) {
        for (int32_t u = 0; u < nu; u++) order->push_back(u);
        return;
    }
    // The hardware deals workgroups to the XCDs round robin (workgroup b on
    // XCD b % 8), each XCD with its own L2.  A unit stages the B rows of one
    // range of its panel's sorted column union.  Units whose columns span at
    // most K / 4 are sorted by the middle of that span and cut into 8 runs of
    // equal tiles; run x goes to XCD x in column order, so the units resident
    // together on one XCD stage nearby B rows and meet them in its L2.  Wider
    // units follow, each on the XCD with the fewest tiles so far; shorter
    // queues end in idle workgroups.
    std::vector<std::pair<int64_t, int32_t>> local;
    std::vector<int32_t> wide;
    int64_t local_tiles = 0;
    for (int32_t u = 0; u < nu; u++) {
        if ((hi[u] - lo[u]) * (kXcds / 2) <= K) {
            local.push_back({lo[u] + hi[u], u});
            local_tiles += units[u].z;
        } else {
            wide.push_back(u);
        }
    }
    std::stable_sort(local.begin(), local.end());
    std::vector<std::vector<int32_t>> q(kXcds);
    std::vector<int64_t> load(kXcds, 0);
    int64_t cum = 0;
    for (const auto& l : local) {
        const int32_t z = units[l.second].z;
        const int32_t x = static_cast<int32_t>(std::min<int64_t>(kXcds - 1, (2 * cum + z) * kXcds / (2 * local_tiles)));
        q[x].push_back(l.second);
        load[x] += z;
        cum += z;
    }
    for (int32_t u : wide) {
        const int32_t x = static_cast<int32_t>(std::min_element(load.begin(), load.end()) - load.begin());
        q[x].push_back(u);
        load[x] += units[u].z;
    }
    size_t len = 0;
    for (const auto& v : q) len = std::max(len, v.size());
    order->assign(len * kXcds, -1);
    for (int32_t x = 0; x < kXcds; x++)
        for (size_t k = 0; k < q[x].size(); k++) (*order)[k * kXcds + x] = q[x][k];
}

bool row_order_on(const RowPlan& p) {
    const char* e = std::getenv("TCA_ROW_ORDER");  // tuning override: 0 = task order
    return p.col_chunks == 1 && p.n_seg >= kXcds * kRowOrderSlots && !(e && std::atoi(e) == 0);
}

void order_row_tasks(const int32_t* colidx, RowPlan* p) {
    p->order.clear();
    constexpr int32_t W = kRowOrderSlots;
    if (!row_order_on(*p)) return;
    // Workgroup b runs on XCD b % 8.  A long row's segments are column
    // ranges of it (columns ascend within a row); sorted by the column of
    // their middle nonzero and cut into 8 runs of equal count, run x goes to
    // XCD x in column order, so the segments resident together on one XCD
    // gather nearby B rows and meet them in its L2.  Wide rows' quarter
    // groups (one workgroup each) keep their places before them, row and
    // multi tasks follow in task order.
    const int32_t nw = p->n_wide, ns = p->n_seg;
    std::vector<std::pair<int32_t, int32_t>> seg(ns);
    for (int32_t i = 0; i < ns; i++) {
        const Int4& t = p->tasks[nw + i];
        seg[i] = {colidx[t.y + (t.z - t.y) / 2], nw + i};
    }
    std::stable_sort(seg.begin(), seg.end());
    for (int32_t i = 0; i < nw; i++) p->order.push_back(i);
    std::vector<size_t> next(kXcds), end(kXcds);
    for (int32_t x = 0; x < kXcds; x++) {
        next[x] = static_cast<size_t>(ns) * x / kXcds;
        end[x] = static_cast<size_t>(ns) * (x + 1) / kXcds;
    }
    for (size_t b = static_cast<size_t>(nw) / W;; b++) {
        bool left = false;
        for (int32_t x = 0; x < kXcds; x++) left = left || next[x] < end[x];
        if (!left) break;
        const size_t x = b % kXcds;
        for (int32_t k = 0; k < W; k++) p->order.push_back(next[x] < end[x] ? seg[next[x]++].second : -1);
    }
    for (int32_t i = nw + ns; i < static_cast<int32_t>(p->tasks.size()); i++) p->order.push_back(i);
    while (p->order.size() % W) p->order.push_back(-1);
}

}  // namespace tca

extern "C" int tca_condense_windows(const int32_t* rowptr, const int32_t* colidx, int32_t M, int32_t nnz,
                                    int32_t win, int64_t* uoff, int32_t* ucols, int32_t* cpos) {
    return tca::api_guard("tca_condense_windows", [&]() -> int {
        using namespace tca;
        if (!rowptr || (nnz > 0 && !colidx) || M < 0 || win < 1 || !uoff)
            return fail(TCA_ERR_INVALID, "tca_condense_windows: bad argument");
        if (rowptr[M] != nnz) return fail(TCA_ERR_INVALID, "tca_condense_windows: rowptr[M] != nnz");
        std::vector<int64_t> off;
        std::vector<int32_t> uc, cp;
        if (cpos) cp.resize(nnz);
        condense(rowptr, colidx, M, win, &off, ucols ? &uc : nullptr, cpos ? &cp : nullptr);
        std::copy(off.begin(), off.end(), uoff);
        if (ucols) std::copy(uc.begin(), uc.end(), ucols);
        if (cpos) std::copy(cp.begin(), cp.end(), cpos);
        return TCA_OK;
    });
}

extern "C" int tca_plan_row_tasks(const int32_t* rowptr, int32_t M, int32_t K, int32_t N, int32_t dtype, int32_t* n_tasks,
                                  int32_t* n_perm, int32_t* n_long, int32_t* tasks, int32_t* perm, int32_t* longrows,
                                  int32_t* geometry) {
    return tca::api_guard("tca_plan_row_tasks", [&]() -> int {
        using namespace tca;
        if (!rowptr || M < 0 || K < 1 || N < 1 || !dtype_ok(dtype) || !n_tasks || !n_perm || !n_long)
            return fail(TCA_ERR_INVALID, "tca_plan_row_tasks: bad argument");
        RowPlan p;
        plan_rows(rowptr, M, N, static_cast<int32_t>(dtype_size(dtype)), {}, default_slices(K, N, dtype), &p);
        if (tasks) {
            if (*n_tasks < static_cast<int32_t>(p.tasks.size()) || *n_perm < static_cast<int32_t>(p.perm.size()) ||
                *n_long < static_cast<int32_t>(p.longrows.size()) || !perm || !longrows)
                return fail(TCA_ERR_INVALID, "tca_plan_row_tasks: output buffers too small");
            if (!p.tasks.empty()) std::copy(&p.tasks[0].x, &p.tasks[0].x + 4 * p.tasks.size(), tasks);
            std::copy(p.perm.begin(), p.perm.end(), perm);
            if (!p.longrows.empty()) std::copy(&p.longrows[0].x, &p.longrows[0].x + 4 * p.longrows.size(), longrows);
        }
        *n_tasks = static_cast<int32_t>(p.tasks.size());
        *n_perm = static_cast<int32_t>(p.perm.size());
        *n_long = static_cast<int32_t>(p.longrows.size());
        if (geometry) {
            geometry[0] = p.elems_per_lane;
            geometry[1] = 1 << p.log_lanes;
            geometry[2] = p.col_chunks;
            geometry[3] = p.seg_len;
            geometry[4] = p.chunk_lanes;
            geometry[5] = p.row_len;
            geometry[6] = p.wide_len;
            geometry[7] = p.multi_max;
        }
        return TCA_OK;
    });
}

extern "C" int tca_plan_mfma_windows(const int32_t* rowptr, const int32_t* colidx, int32_t M, int32_t N,
                                     int32_t dtype, uint32_t flags, int32_t* n_windows, int32_t* n_steps,
                                     int64_t* n_entries, int32_t* windows, int32_t* ucols, int32_t* eoff,
                                     uint32_t* entries) {
    return tca::api_guard("tca_plan_mfma_windows", [&]() -> int {
        using namespace tca;
        if (!rowptr || M < 0 || N < 1 || !dtype_ok(dtype) || !n_windows || !n_steps || !n_entries)
            return fail(TCA_ERR_INVALID, "tca_plan_mfma_windows: bad argument");
        MfmaPlan p;
        const char* md = std::getenv("TCA_MFMA_MIN_DENSITY");
        plan_mfma(rowptr, colidx, M, N, dtype, (flags & TCA_PLAN_FORCE_MFMA) != 0, (flags & TCA_PLAN_NO_MFMA) != 0,
                  md ? std::atof(md) : kMfmaMinDensity, mfma_shape(flags), &p);
        const int32_t steps = static_cast<int32_t>(p.eoff.size()) - 1;
        if (windows) {
            if (*n_windows < static_cast<int32_t>(p.windows.size()) || *n_steps < steps ||
                *n_entries < static_cast<int64_t>(p.entries.size()) || !ucols || !eoff || !entries)
                return fail(TCA_ERR_INVALID, "tca_plan_mfma_windows: output buffers too small");
            if (!p.windows.empty()) std::copy(&p.windows[0].x, &p.windows[0].x + 4 * p.windows.size(), windows);
            std::copy(p.ucols.begin(), p.ucols.end(), ucols);
            std::copy(p.eoff.begin(), p.eoff.end(), eoff);
            std::copy(p.entries.begin(), p.entries.end(), entries);
        }
        *n_windows = static_cast<int32_t>(p.windows.size());
        *n_steps = steps;
        *n_entries = static_cast<int64_t>(p.entries.size());
        return TCA_OK;
    });
}

extern "C" int tca_plan_launch_orders(const int32_t* rowptr, const int32_t* colidx, int32_t M, int32_t K, int32_t N,
                                      int32_t dtype, uint32_t flags, int32_t* n_blocks, int32_t* panel_order,
                                      int32_t* n_tasks, int32_t* tasks, int32_t* n_slots, int32_t* row_order) {
    return tca::api_guard("tca_plan_launch_orders", [&]() -> int {
        using namespace tca;
        if (!rowptr || !colidx || M < 0 || K < 1 || N < 1 || !dtype_ok(dtype) || !n_blocks || !n_tasks || !n_slots)
            return fail(TCA_ERR_INVALID, "tca_plan_launch_orders: bad argument");
        MfmaPlan mp;
        const char* md = std::getenv("TCA_MFMA_MIN_DENSITY");
        plan_mfma(rowptr, colidx, M, N, dtype, (flags & TCA_PLAN_FORCE_MFMA) != 0, (flags & TCA_PLAN_NO_MFMA) != 0,
                  md ? std::atof(md) : kMfmaMinDensity, mfma_shape(flags), &mp);
        PanelPlan pp;
        plan_panels_routed(rowptr, colidx, M, K, N, dtype, flags, mp.row_mfma, &pp);
        std::vector<uint8_t> skip(M, 0);
        for (int32_t r = 0; r < M; r++) skip[r] = (!mp.row_mfma.empty() && mp.row_mfma[r]) || pp.row_panel[r];
        RowPlan rp;
        plan_rows(rowptr, M, N, static_cast<int32_t>(dtype_size(dtype)), skip, default_slices(K, N, dtype), &rp);
        order_row_tasks(colidx, &rp);
        if (panel_order) {
            if (*n_blocks < static_cast<int32_t>(pp.order.size()) || *n_tasks < static_cast<int32_t>(rp.tasks.size()) ||
                *n_slots < static_cast<int32_t>(rp.order.size()) || !tasks || !row_order)
                return fail(TCA_ERR_INVALID, "tca_plan_launch_orders: output buffers too small");
            std::copy(pp.order.begin(), pp.order.end(), panel_order);
            for (size_t t = 0; t < rp.tasks.size(); t++) {
                tasks[4 * t] = rp.tasks[t].x;
                tasks[4 * t + 1] = rp.tasks[t].y;
                tasks[4 * t + 2] = rp.tasks[t].z;
                tasks[4 * t + 3] = rp.tasks[t].w;
            }
            std::copy(rp.order.begin(), rp.order.end(), row_order);
        }
        *n_blocks = static_cast<int32_t>(pp.order.size());
        *n_tasks = static_cast<int32_t>(rp.tasks.size());
        *n_slots = static_cast<int32_t>(rp.order.size());
        return TCA_OK;
    });
}

extern "C" int tca_plan_panels(const int32_t* rowptr, const int32_t* colidx, int32_t M, int32_t K, int32_t N,
                               int32_t dtype, uint32_t flags, int64_t* sizes, int32_t* rows, int32_t* cols,
                               uint8_t* width, uint8_t* cnt, uint8_t* pos, int32_t* units, int32_t* panel_units,
                               int32_t* ustart, int32_t* longrows) {
    return tca::api_guard("tca_plan_panels", [&]() -> int {
        using namespace tca;
        if (!rowptr || !colidx || M < 0 || K < 1 || N < 1 || !dtype_ok(dtype) || !sizes)
            return fail(TCA_ERR_INVALID, "tca_plan_panels: bad argument");
        MfmaPlan mp;
        const char* md = std::getenv("TCA_MFMA_MIN_DENSITY");
        plan_mfma(rowptr, colidx, M, N, dtype, (flags & TCA_PLAN_FORCE_MFMA) != 0, (flags & TCA_PLAN_NO_MFMA) != 0,
                  md ? std::atof(md) : kMfmaMinDensity, mfma_shape(flags), &mp);
        PanelPlan p;
        plan_panels_routed(rowptr, colidx, M, K, N, dtype, flags, mp.row_mfma, &p);
        const int64_t stride = static_cast<int64_t>(p.waves) * kPanelCntRows * 4;
        const int64_t sz[16] = {p.n_panels, p.n_tiles(), static_cast<int64_t>(p.units.size()),
                                static_cast<int64_t>(p.longrows.size()), p.R, p.P, p.waves, p.rpg, p.elems, p.chunks,
                                p.nnz, p.staged, p.n_segments, p.n_rows, stride, kPanelMaxDword};
        std::copy(sz, sz + 16, sizes);
        if (!rows) return TCA_OK;
        if (!cols || !width || !cnt || !pos || !units || !panel_units || !ustart || !longrows)
            return fail(TCA_ERR_INVALID, "tca_plan_panels: missing output array");
        std::copy(p.rows.begin(), p.rows.end(), rows);
        std::copy(p.cols.begin(), p.cols.end(), cols);
        std::copy(p.width.begin(), p.width.end(), width);
        std::copy(p.cnt.begin(), p.cnt.end(), cnt);
        if (!p.pos.empty()) std::copy(p.pos.begin(), p.pos.begin() + rowptr[M], pos);
        else std::fill(pos, pos + rowptr[M], 0);
        for (size_t u = 0; u < p.units.size(); u++) {
            units[4 * u] = p.units[u].x;
            units[4 * u + 1] = p.units[u].y;
            units[4 * u + 2] = p.units[u].z;
            units[4 * u + 3] = p.units[u].w;
        }
        std::copy(p.panel_units.begin(), p.panel_units.end(), panel_units);
        std::copy(p.ustart.begin(), p.ustart.end(), ustart);
        for (size_t u = 0; u < p.longrows.size(); u++) {
            longrows[4 * u] = p.longrows[u].x;
            longrows[4 * u + 1] = p.longrows[u].y;
            longrows[4 * u + 2] = p.longrows[u].z;
            longrows[4 * u + 3] = p.longrows[u].w;
        }
        return TCA_OK;
    });
}
