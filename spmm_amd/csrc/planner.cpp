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
    // Work per wavefront task: about nnz / 16384 nonzeros (two resident
    // wavefronts on each of 256 CUs x 4 SIMDs x 8 slots, so long rows do
    // not leave a latency tail), a power of two of at least 256 nonzeros and
    // 2 rounds of slots * kUnroll loads, at most 32 rounds.  (Shorter tasks
    // cost more in partial sums than they gain in balance: on MI355X the
    // 4096 x 4096 config-1 matrix runs 44 us at 256 and 47 us at 64.)
    const int64_t round = static_cast<int64_t>(slots) * kUnroll;
    int64_t target = next_pow2(std::max<int64_t>(nnz / 16384, 1));
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
    for (i = first_row; i < rows.size() && len(rows[i]) > p->multi_max; i++) {
        const int32_t r = rows[i];
        p->tasks.push_back({r, rowptr[r], rowptr[r + 1], kTaskRow});
    }
    p->n_rowtasks = static_cast<int32_t>(p->tasks.size()) - p->n_seg - p->n_wide;
    // Short rows: groups of `slots` rows of similar length.
    const size_t first_multi = p->tasks.size();
    for (; i < rows.size(); i += slots) {
        const int32_t cnt = static_cast<int32_t>(std::min<size_t>(slots, rows.size() - i));
        p->tasks.push_back({static_cast<int32_t>(p->perm.size()), cnt, len(rows[i]), kTaskMulti});
        for (int32_t k = 0; k < cnt; k++) p->perm.push_back(rows[i + k]);
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

void plan_mfma24(const MfmaPlan& m, const int32_t* rowptr, const int32_t* colidx, Mfma24Plan* p) {
    constexpr int kWin = 128, kStep64 = 64;
    *p = Mfma24Plan();
    const size_t nw = m.windows.size();
    // per window: the grouped order of its condensed columns
    std::vector<std::vector<int32_t>> order(nw);
    std::vector<int64_t> pads(nw, 0);
#pragma omp parallel for schedule(dynamic, 1)
    for (size_t w = 0; w < nw; w++) {
        const Int4 win = m.windows[w];
        const int32_t r0 = win.x, r1 = std::min<int32_t>(r0 + kWin, static_cast<int32_t>(m.row_mfma.size()));
        // the window's column union (the condensed columns, ascending) and,
        // per column, the rows holding it
        std::vector<int32_t> u;
        for (int32_t s = 0; s < win.y; s++)
            for (int32_t k = 0; k < 32; k++) {
                const int32_t c = m.ucols[static_cast<size_t>(win.z + s) * 32 + k];
                if (c >= 0) u.push_back(c);
            }
        std::vector<int32_t> first(u.size() + 1, 0), rowsof;
        {
            std::vector<int32_t> cnt(u.size(), 0);
            for (int32_t r = r0; r < r1; r++)
                for (int32_t j = rowptr[r]; j < rowptr[r + 1]; j++)
                    cnt[std::lower_bound(u.begin(), u.end(), colidx[j]) - u.begin()]++;
            for (size_t i = 0; i < u.size(); i++) first[i + 1] = first[i] + cnt[i];
            rowsof.resize(first.back());
            std::vector<int32_t> fill(first.begin(), first.end() - 1);
            for (int32_t r = r0; r < r1; r++)
                for (int32_t j = rowptr[r]; j < rowptr[r + 1]; j++)
                    rowsof[fill[std::lower_bound(u.begin(), u.end(), colidx[j]) - u.begin()]++] = r - r0;
        }
        // Greedy: each column joins the first open group (of the most recent
        // ones) in which none of its rows already has two entries; a group
        // closes at 4 columns; a column fitting none opens a new group.
        constexpr int kOpen = 16;
        struct Group {
            int32_t c[4];
            int32_t n;
            uint8_t cnt[kWin];
        };
        std::vector<Group> groups;
        std::vector<int32_t> open;  // indices into groups, not yet full
        for (size_t i = 0; i < u.size(); i++) {
            int32_t g = -1;
            for (int32_t o : open) {
                bool ok = true;
                for (int32_t t = first[i]; t < first[i + 1] && ok; t++) ok = groups[o].cnt[rowsof[t]] < 2;
                if (ok) {
                    g = o;
                    break;
                }
            }
            if (g < 0) {
                groups.push_back(Group{});
                std::memset(&groups.back(), 0, sizeof(Group));
                g = static_cast<int32_t>(groups.size()) - 1;
                open.push_back(g);
                if (open.size() > kOpen) open.erase(open.begin());  // oldest stays partly empty (padding)
            }
            Group& G = groups[g];
            G.c[G.n++] = static_cast<int32_t>(i);
            for (int32_t t = first[i]; t < first[i + 1]; t++) G.cnt[rowsof[t]]++;
            if (G.n == 4) open.erase(std::find(open.begin(), open.end(), g));
        }
        std::vector<int32_t>& ord = order[w];
        for (const Group& G : groups)
            for (int32_t k = 0; k < 4; k++) ord.push_back(k < G.n ? u[G.c[k]] : -1);
        while (ord.size() % kStep64) ord.push_back(-1);
        pads[w] = static_cast<int64_t>(ord.size() - u.size());
    }
    // global steps, B rows, compressed positions and index words
    int32_t gstep = 0;
    std::vector<std::vector<std::pair<uint32_t, int32_t>>> wpos(nw);
    for (size_t w = 0; w < nw; w++) {
        const Int4 win = m.windows[w];
        const int32_t steps = static_cast<int32_t>(order[w].size() / kStep64);
        p->windows.push_back({win.x, steps, gstep, win.w});
        p->cols.insert(p->cols.end(), order[w].begin(), order[w].end());
        p->pad_cols += pads[w];
        gstep += steps;
    }
    p->idx.assign(static_cast<size_t>(gstep) * 8 * 64, 0x44444444u);
#pragma omp parallel for schedule(dynamic, 1)
    for (size_t w = 0; w < nw; w++) {
        const Int4 win = p->windows[w];
        const std::vector<int32_t>& ord = order[w];
        // condensed position of each column of the window
        std::vector<std::pair<int32_t, int32_t>> at;  // (column, position)
        for (size_t q = 0; q < ord.size(); q++)
            if (ord[q] >= 0) at.emplace_back(ord[q], static_cast<int32_t>(q));
        std::sort(at.begin(), at.end());
        const int32_t r1 = std::min<int32_t>(win.x + kWin, static_cast<int32_t>(m.row_mfma.size()));
        for (int32_t r = win.x; r < r1; r++) {
            // this row's entries by condensed position
            std::vector<std::pair<int32_t, int32_t>> e;  // (position, nonzero)
            for (int32_t j = rowptr[r]; j < rowptr[r + 1]; j++)
                e.emplace_back(std::lower_bound(at.begin(), at.end(), std::make_pair(colidx[j], -1))->second, j);
            std::sort(e.begin(), e.end());
            const int32_t rr = r - win.x, rb = rr / 16;
            for (size_t a = 0; a < e.size();) {
                const int32_t grp = e[a].first / 4;
                size_t b = a;
                while (b < e.size() && e[b].first / 4 == grp) b++;
                // b - a <= 2 by construction
                int32_t p0, p1, slot0 = -1, slot1 = -1;
                if (b - a == 2) {
                    p0 = e[a].first % 4, p1 = e[a + 1].first % 4, slot0 = static_cast<int32_t>(a),
                    slot1 = static_cast<int32_t>(a + 1);
                } else {
                    const int32_t q = e[a].first % 4;
                    if (q == 3) p0 = 2, p1 = 3, slot1 = static_cast<int32_t>(a);
                    else p0 = q, p1 = q + 1, slot0 = static_cast<int32_t>(a);
                }
                const int32_t pos = grp * 4;
                const int32_t step = pos / kStep64, lc = pos % kStep64;
                const int32_t lane = rr % 16 + 16 * (lc / 16), G = (lc % 16) / 4;
                const size_t word = (static_cast<size_t>(win.z + step) * 8 + rb) * 64 + lane;
                const uint32_t nib = static_cast<uint32_t>(p0 | (p1 << 2));
                uint32_t v = p->idx[word] & 0xffffu;
                v = (v & ~(0xfu << (4 * G))) | (nib << (4 * G));
                p->idx[word] = v | (v << 16);
                const size_t half = word * 8 + 2 * G;
                if (slot0 >= 0) wpos[w].emplace_back(static_cast<uint32_t>(half), e[slot0].second);
                if (slot1 >= 0) wpos[w].emplace_back(static_cast<uint32_t>(half + 1), e[slot1].second);
                a = b;
            }
        }
        std::sort(wpos[w].begin(), wpos[w].end());
    }
    for (auto& v : wpos) p->pos.insert(p->pos.end(), v.begin(), v.end());
}

}  // namespace tca

extern "C" int tca_condense_windows(const int32_t* rowptr, const int32_t* colidx, int32_t M, int32_t nnz,
                                    int32_t win, int64_t* uoff, int32_t* ucols, int32_t* cpos) {
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
}

extern "C" int tca_plan_row_tasks(const int32_t* rowptr, int32_t M, int32_t K, int32_t N, int32_t dtype, int32_t* n_tasks,
                                  int32_t* n_perm, int32_t* n_long, int32_t* tasks, int32_t* perm, int32_t* longrows,
                                  int32_t* geometry) {
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
}

extern "C" int tca_plan_mfma_windows(const int32_t* rowptr, const int32_t* colidx, int32_t M, int32_t N,
                                     int32_t dtype, uint32_t flags, int32_t* n_windows, int32_t* n_steps,
                                     int64_t* n_entries, int32_t* windows, int32_t* ucols, int32_t* eoff,
                                     uint32_t* entries) {
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
}
