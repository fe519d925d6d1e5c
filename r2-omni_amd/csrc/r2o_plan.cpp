// Work-item planner of the split-K decode launch (host code only; no GPU work, callable on any
// machine).  The reference launches one program per BLOCK_N tile of every pool and counts those
// tiles while preparing the executor (triton_fourq_splitk.py:1772-1817); this build instead splits
// each (request, KV head, pool segment) run of 32-token tiles into work items of about equal
// weighted cost, a bounded number per launch, and resolves each item's base pointers here, so a
// re-plan after a flush costs tens of microseconds of host time.
#include <algorithm>
#include <cmath>
#include <queue>
#include <utility>
#include <vector>

#include "r2o_sspa.h"

namespace {

constexpr int64_t kTile = 32;
constexpr int kKindRecent = 3;

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

struct Split {
    int64_t first, size;  // in tiles, relative to the run's first tile
};

// The items of one run: multiples of `w` tiles each but the last; with late_share < 1 the second
// half of the items gets that share of the first half's work.
void split_run(int64_t nt, int64_t n_items, double late_share, int64_t w, std::vector<Split>& out) {
    out.clear();
    if (late_share >= 1.0 || n_items < 2) {
        const int64_t n = ceil_div(ceil_div(nt, n_items), w) * w;
        for (int64_t f = 0; f < nt; f += n) out.push_back({f, std::min(n, nt - f)});
        return;
    }
    const int64_t big = ceil_div(n_items, 2), small = n_items - big;
    const double x = (double)nt / ((double)big + late_share * (double)small);
    const int64_t bsize = ceil_div((int64_t)std::nearbyint(x), w) * w;  // round half to even
    int64_t f = 0;
    for (int64_t k = 0; k < n_items; ++k) {
        if (f >= nt) break;
        int64_t size = k < big ? bsize : ceil_div(ceil_div(nt - f, n_items - k), w) * w;
        size = std::min(size, nt - f);
        out.push_back({f, size});
        f += size;
    }
    if (f < nt) out.back().size += nt - f;  // rounding left a remainder: the last item takes it
}

// A run's tiles and valid range: tile0 >= 0, aligned to a tile, tile0 <= lo < hi <= tile0 + 32 * ntiles.
// With the request descriptors, the tiles must lie inside the request's K arena (or ring) and the
// V rows [lo - v_delta, hi - v_delta) inside the run's V pool: the partial kernel reads whole K tiles
// and clamps V rows to the valid range, at the base pointers the planner computes from these.
bool run_in_bounds(const r2o_plan_run& r, const r2o_request_desc* reqs, int64_t k_format) {
    const int64_t end = r.tile0 + kTile * r.ntiles;
    if (r.tile0 < 0 || r.tile0 % kTile || r.lo < r.tile0 || r.hi <= r.lo || r.hi > end) return false;
    if (!reqs) return true;
    const r2o_request_desc& d = reqs[r.req];
    if (r.kind == kKindRecent) return r.v_delta == 0 && end <= d.recent_capacity;
    if (end > d.k_capacity || (k_format != R2O_K_BF16 && (!d.k_operands || d.k_superblocks <= 0))) return false;
    const int64_t stride = r.kind == 0 ? d.fp_stride : (r.kind == 1 ? d.i4_stride : d.i2_stride);
    return r.lo - r.v_delta >= 0 && r.hi - r.v_delta <= stride;
}

}  // namespace

extern "C" int r2o_plan_work_items(const r2o_plan_run* runs, int64_t n_runs, const r2o_plan_config* cfg,
                                   const r2o_request_desc* reqs, int64_t n_reqs, int64_t k_format,
                                   int64_t int2_group, r2o_work_item* items, int64_t max_items,
                                   int32_t* group_begin, int64_t n_groups, int64_t* n_items) {
    if (!runs || !cfg || !items || !group_begin || !n_items || n_runs <= 0 || n_groups <= 0) return R2O_EINVAL;
    if (cfg->waves_per_item <= 0 || cfg->min_tiles_per_item <= 0 || cfg->tiles_per_item <= 0 ||
        cfg->blocks_per_cu <= 0)
        return R2O_EINVAL;
    if (n_reqs <= 0 || n_groups % n_reqs) return R2O_EINVAL;
    const int64_t hkv = n_groups / n_reqs;
    if (reqs && !(k_format == R2O_K_INT4 || k_format == R2O_K_BF16 || k_format == R2O_K_INT2)) return R2O_EINVAL;
    const bool group_ok = int2_group == 32 || int2_group == 64 || int2_group == 128;
    int64_t total_tiles = 0;
    for (int64_t i = 0; i < n_runs; ++i) {
        const r2o_plan_run& r = runs[i];
        if (r.kind < 0 || r.kind > kKindRecent || r.ntiles < 1 || r.req < 0 || r.req >= n_reqs) return R2O_EINVAL;
        if (r.kvh < 0 || r.kvh >= hkv) return R2O_EINVAL;
        if (r.kind == 2 && !group_ok) return R2O_EINVAL;  // every INT2-V item carries its group size
        if (!run_in_bounds(r, reqs, k_format)) return R2O_EINVAL;
        total_tiles += r.ntiles;
    }
    // Water-filling: one more item for the run whose items are the most expensive (ties: the
    // earlier run) until the launch's slots are used up or no run can be split further.
    const int64_t cus = std::max<int64_t>(1, cfg->num_cus);
    const int64_t target =
        std::min(cfg->blocks_per_cu * cus, std::max(cus, total_tiles / cfg->tiles_per_item));
    std::vector<int64_t> counts(n_runs, 1);
    auto item_cost = [&](int64_t i) {
        const int64_t per = ceil_div(runs[i].ntiles, counts[i]);
        return (double)(ceil_div(per, cfg->waves_per_item) * cfg->waves_per_item) * cfg->tile_cost[runs[i].kind];
    };
    using Entry = std::pair<double, int64_t>;  // (cost, run): the largest cost first, then the lower run index
    auto later = [](const Entry& a, const Entry& b) { return a.first < b.first || (a.first == b.first && a.second > b.second); };
    std::priority_queue<Entry, std::vector<Entry>, decltype(later)> heap(later);
    for (int64_t i = 0; i < n_runs; ++i) heap.push({item_cost(i), i});
    int64_t total = n_runs;
    while (total < target && !heap.empty()) {
        const int64_t i = heap.top().second;
        heap.pop();
        if (ceil_div(runs[i].ntiles, counts[i] + 1) < cfg->min_tiles_per_item) continue;  // smallest useful size
        counts[i] += 1;
        total += 1;
        heap.push({item_cost(i), i});
    }
    int first_kind = -1;
    bool uniform = true;
    for (int64_t i = 0; i < n_runs; ++i) {
        if (runs[i].kind == kKindRecent) continue;
        if (first_kind < 0) first_kind = (int)runs[i].kind;
        else if (runs[i].kind != first_kind) uniform = false;
    }
    const double late_share = (uniform && total > cus) ? cfg->late_share : 1.0;

    // Items in (request, KV head) order, which numbers their partial slots; then launched largest first.
    std::vector<r2o_work_item> planned;
    planned.reserve(total);
    // Group g = request g / hkv, KV head g % hkv: the runs come in group order, every group has one.
    int64_t group = 0;
    group_begin[0] = 0;
    std::vector<Split> parts;
    for (int64_t i = 0; i < n_runs; ++i) {
        const r2o_plan_run& r = runs[i];
        const int64_t gid = r.req * hkv + r.kvh;
        if (gid != group) {
            if (gid != group + 1 || i == 0) return R2O_EINVAL;
            group = gid;
            group_begin[group] = (int32_t)planned.size();
        }
        split_run(r.ntiles, counts[i], late_share, cfg->waves_per_item, parts);
        for (const Split& s : parts) {
            r2o_work_item it{};
            it.req = r.req;
            it.kvh = r.kvh;
            it.kind = r.kind;
            it.tile0 = r.tile0 + kTile * s.first;
            it.ntiles = s.size;
            it.lo = r.lo;
            it.hi = r.hi;
            it.v_delta = r.v_delta;
            it.slot = (int64_t)planned.size();
            planned.push_back(it);
        }
    }
    if (group + 1 != n_groups) return R2O_EINVAL;
    group_begin[n_groups] = (int32_t)planned.size();
    if ((int64_t)planned.size() > max_items) return R2O_EINVAL;
    std::stable_sort(planned.begin(), planned.end(), [&](const r2o_work_item& a, const r2o_work_item& b) {
        return (double)a.ntiles * cfg->tile_cost[a.kind] > (double)b.ntiles * cfg->tile_cost[b.kind];
    });

    // Base pointers of each item's head (the pointer arithmetic the kernel would otherwise do).
    const int64_t k_row = k_format == R2O_K_INT4 ? 64 : (k_format == R2O_K_INT2 ? 32 : 256);
    const int64_t groups = group_ok ? 128 / int2_group : 1;  // INT2-V scale / zero columns per token
    for (r2o_work_item& it : planned) {
        if (it.kind == 2) it.v_group = int2_group;
        if (!reqs) continue;
        const r2o_request_desc& d = reqs[it.req];
        const int64_t h = it.kvh;
        if (it.kind == kKindRecent) {
            const int64_t row = h * d.recent_capacity * 256;
            it.k_base = reinterpret_cast<const unsigned char*>(d.recent_k) + row;
            it.v_base = reinterpret_cast<const unsigned char*>(d.recent_v) + row;
            it.ring_length = d.recent_length;
            continue;
        }
        it.k_base = d.k_packed + h * d.k_capacity * k_row;
        it.k_ops = d.k_operands ? d.k_operands + h * d.k_superblocks * 128 : nullptr;
        if (it.kind == 0) {
            it.v_base = reinterpret_cast<const unsigned char*>(d.fp_v) + h * d.fp_stride * 256;
        } else if (it.kind == 1) {
            it.v_base = d.i4_v + h * d.i4_stride * 64;
            it.v_scale = d.i4_scale + h * d.i4_stride;
        } else {
            it.v_base = d.i2_v + h * d.i2_stride * 32;
            it.v_scale = d.i2_scale + h * d.i2_stride * groups;
            it.v_zero = d.i2_zero + h * d.i2_stride * groups;
        }
    }
    std::copy(planned.begin(), planned.end(), items);
    *n_items = (int64_t)planned.size();
    return R2O_OK;
}
