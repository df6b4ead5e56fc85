// Python bindings of the CPU oracle — TEST INFRASTRUCTURE ONLY.
// Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.
#include <array>

#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <omp.h>

#include "cptc_oracle.hpp"
#include "cptc_oracle_nd.hpp"

namespace py = pybind11;
using namespace oracle;

template <class T>
using arr = py::array_t<T, py::array::c_style | py::array::forcecast>;

template <class T>
std::vector<T> vec(const arr<T>& a)
{
    return std::vector<T>(a.data(), a.data() + a.size());
}

template <class T>
arr<T> np(const std::vector<T>& v)
{
    arr<T> a(v.size());
    if (!v.empty()) std::memcpy(a.mutable_data(), v.data(), v.size() * sizeof(T));
    return a;
}

static void dims_from(const py::sequence& d, size_t out[3])
{
    for (int m = 0; m < 3; ++m) out[m] = d[m].cast<size_t>();
}

static Coo3 coo_from(arr<int32_t> m0, arr<int32_t> m1, arr<int32_t> m2, arr<double> v,
                     py::sequence dims)
{
    Coo3 t;
    t.m0 = vec(m0);
    t.m1 = vec(m1);
    t.m2 = vec(m2);
    t.val = vec(v);
    dims_from(dims, t.dims);
    return t;
}

static py::dict part_to_dict(const Partition3& p)
{
    py::dict d;
    d["cutoff"] = p.cutoff;
    std::vector<int32_t> t4;
    std::vector<uint64_t> off;
    for (const Tile& t : p.tiles)
    {
        t4.insert(t4.end(), {t.b[0], t.b[1], t.b[2], t.nnz});
        off.push_back(t.off);
    }
    off.push_back(p.pool_lid.size());
    d["tiles"] = np(t4).attr("reshape")(py::make_tuple(-1, 4));
    d["pool_off"] = np(off);
    d["pool_lid"] = np(p.pool_lid);
    d["pool_val"] = np(p.pool_val);
    d["sp_i"] = np(p.sp_i);
    d["sp_j"] = np(p.sp_j);
    d["sp_k"] = np(p.sp_k);
    d["sp_val"] = np(p.sp_val);
    return d;
}

static Partition3 part_from_dict(const py::dict& d)
{
    Partition3 p;
    p.cutoff = d["cutoff"].cast<int>();
    auto t4 = d["tiles"].cast<arr<int32_t>>();
    auto off = d["pool_off"].cast<arr<uint64_t>>();
    const size_t nt = t4.size() / 4;
    for (size_t t = 0; t < nt; ++t)
    {
        Tile tl;
        for (int q = 0; q < 3; ++q) tl.b[q] = t4.data()[t * 4 + q];
        tl.nnz = t4.data()[t * 4 + 3];
        tl.off = off.data()[t];
        p.tiles.push_back(tl);
    }
    p.pool_lid = vec(d["pool_lid"].cast<arr<int32_t>>());
    p.pool_val = vec(d["pool_val"].cast<arr<double>>());
    return p;
}

static py::list view_to_list(const View3& v)
{
    py::list l;
    for (int m = 0; m < 3; ++m)
    {
        py::dict d;
        d["coords"] = np(v.coords[m]);
        d["vals"] = np(v.vals[m]);
        d["blk_row"] = np(v.blk_row[m]);
        d["blk_start"] = np(v.blk_start[m]);
        d["blk_cnt"] = np(v.blk_cnt[m]);
        l.append(d);
    }
    return l;
}

static View3 view_from_list(const py::list& l)
{
    View3 v;
    for (int m = 0; m < 3; ++m)
    {
        py::dict d = l[m];
        v.coords[m] = vec(d["coords"].cast<arr<uint64_t>>());
        v.vals[m] = vec(d["vals"].cast<arr<double>>());
        v.blk_row[m] = vec(d["blk_row"].cast<arr<uint32_t>>());
        v.blk_start[m] = vec(d["blk_start"].cast<arr<uint32_t>>());
        v.blk_cnt[m] = vec(d["blk_cnt"].cast<arr<uint32_t>>());
        v.nnz = v.vals[m].size();
    }
    return v;
}


static CooN coon_from(arr<uint32_t> coords, arr<double> vals, py::sequence dims)
{
    CooN t;
    t.N = int(py::len(dims));
    for (int m = 0; m < t.N; ++m) t.dims.push_back(dims[m].cast<size_t>());
    const size_t nnz = vals.size();
    t.val = vec(vals);
    t.c.resize(t.N);
    for (int m = 0; m < t.N; ++m)
        t.c[m].assign(coords.data() + size_t(m) * nnz, coords.data() + size_t(m + 1) * nnz);
    return t;
}

static arr<uint32_t> coords_np(const CooN& t)
{
    const size_t nnz = t.nnz();
    arr<uint32_t> a(std::vector<ssize_t>{ssize_t(t.N), ssize_t(nnz)});
    for (int m = 0; m < t.N; ++m)
        if (nnz) std::memcpy(a.mutable_data() + size_t(m) * nnz, t.c[m].data(), nnz * 4);
    return a;
}

static std::vector<std::vector<double>> flist(py::list F)
{
    std::vector<std::vector<double>> out;
    for (auto f : F) out.push_back(vec(f.cast<arr<double>>()));
    return out;
}

static py::list flist_np(const std::vector<std::vector<double>>& F)
{
    py::list l;
    for (auto& f : F) l.append(np(f));
    return l;
}

static py::dict units_to_dict(const UnitsN& u)
{
    py::dict d;
    d["cutoff"] = u.cutoff;
    d["inner"] = py::make_tuple(u.inner[0], u.inner[1], u.inner[2]);
    d["unit6"] = np(u.unit6).attr("reshape")(py::make_tuple(-1, 6));
    d["outer_coords"] = np(u.outer_coords);
    d["lid"] = np(u.lid);
    d["val"] = np(u.val);
    d["is_dense"] = np(u.is_dense);
    return d;
}

static UnitsN units_from_dict(const py::dict& d, int N)
{
    UnitsN u;
    u.cutoff = d["cutoff"].cast<int>();
    if (d.contains("inner"))
    {
        const auto in = d["inner"].cast<std::array<int, 3>>();
        for (int x = 0; x < 3; ++x) u.inner[x] = in[x];
    }
    for (int m = 0; m < N; ++m)
        if (m != u.inner[0] && m != u.inner[1] && m != u.inner[2]) u.outer.push_back(m);
    u.unit6 = vec(d["unit6"].cast<arr<uint32_t>>());
    u.outer_coords = vec(d["outer_coords"].cast<arr<uint32_t>>());
    u.lid = vec(d["lid"].cast<arr<uint32_t>>());
    u.val = vec(d["val"].cast<arr<double>>());
    u.is_dense = vec(d["is_dense"].cast<arr<uint8_t>>());
    return u;
}

static py::list viewn_to_list(const ViewN& v)
{
    py::list l;
    for (size_t n = 0; n < v.sv.size(); ++n)
    {
        py::dict d;
        d["scoords"] = np(v.sc[n]);
        d["vals"] = np(v.sv[n]);
        d["skip"] = np(v.skip[n]);
        d["row"] = np(v.row[n]);
        d["start"] = np(v.start[n]);
        d["cnt"] = np(v.cnt[n]);
        d["single"] = np(v.single[n]);
        l.append(d);
    }
    return l;
}

static ViewN viewn_from_list(const py::list& l)
{
    ViewN v;
    for (auto item : l)
    {
        py::dict d = item.cast<py::dict>();
        v.sc.push_back(vec(d["scoords"].cast<arr<uint32_t>>()));
        v.sv.push_back(vec(d["vals"].cast<arr<double>>()));
        v.skip.push_back(vec(d["skip"].cast<arr<uint8_t>>()));
        v.row.push_back(vec(d["row"].cast<arr<uint32_t>>()));
        v.start.push_back(vec(d["start"].cast<arr<uint32_t>>()));
        v.cnt.push_back(vec(d["cnt"].cast<arr<uint32_t>>()));
        v.single.push_back(vec(d["single"].cast<arr<uint8_t>>()));
    }
    return v;
}

struct PyAls3
{
    View3 residual, dense_view;
    Partition3 tiles;
    bool has_dv = false, has_tiles = false;
    Als3State st;
    double x_sq = 0.0;

    Als3Input input() const
    {
        Als3Input in;
        in.residual = &residual;
        in.dense_view = has_dv ? &dense_view : nullptr;
        in.tiles = has_tiles ? &tiles : nullptr;
        in.x_sq = x_sq;
        return in;
    }
};

PYBIND11_MODULE(cptc_oracle, m)
{
    m.doc() = "CPU oracle of the cpTC CP-ALS hot path (test infrastructure only)";

    m.def("set_threads", [](int n) { omp_set_num_threads(n); });
    m.def("max_threads", []() { return omp_get_max_threads(); });
    m.def("set_num_cus", &set_num_cus);

    m.def("load_tns3", [](const std::string& path) {
        Coo3 t;
        if (!load_tns3(path, t)) throw std::runtime_error("cannot open " + path);
        return py::make_tuple(np(t.m0), np(t.m1), np(t.m2), np(t.val),
                              py::make_tuple(t.dims[0], t.dims[1], t.dims[2]));
    });

    m.def("cadr3", [](arr<int32_t> m0, arr<int32_t> m1, arr<int32_t> m2, py::sequence dims) {
        Coo3 t = coo_from(m0, m1, m2, arr<double>(0), dims);
        t.val.resize(t.m0.size());
        std::vector<int32_t> p[3];
        cadr3(t, p);
        return py::make_tuple(np(p[0]), np(p[1]), np(p[2]));
    });

    m.def("init_factors3", [](py::sequence dims, int R, unsigned seed) {
        size_t d[3];
        dims_from(dims, d);
        std::vector<double> F[3];
        init_factors3(d, R, seed, F);
        return py::make_tuple(np(F[0]), np(F[1]), np(F[2]));
    });

    m.def("partition3", [](arr<int32_t> m0, arr<int32_t> m1, arr<int32_t> m2, arr<double> v,
                           py::sequence dims, double thr) {
        Coo3 t = coo_from(m0, m1, m2, v, dims);
        Partition3 p;
        partition3(t, thr, p);
        return part_to_dict(p);
    });

    m.def("views3", [](arr<uint32_t> i, arr<uint32_t> j, arr<uint32_t> k, arr<double> v,
                       py::sequence dims) {
        size_t d[3];
        dims_from(dims, d);
        View3 out;
        views3(vec(i), vec(j), vec(k), vec(v), d, out);
        return view_to_list(out);
    });

    m.def("dense_views3", [](py::dict part, py::sequence dims) {
        size_t d[3];
        dims_from(dims, d);
        Partition3 p = part_from_dict(part);
        View3 out;
        dense_views3(p, d, out);
        return view_to_list(out);
    });

    m.def("mttkrp3_view", [](py::list view, int mode, arr<double> A, arr<double> B,
                             arr<double> C, int R, size_t dim) {
        View3 v = view_from_list(view);
        std::vector<double> out(dim * size_t(R), 0.0);
        mttkrp3_view(v, mode, A.data(), B.data(), C.data(), R, out.data());
        return np(out);
    });

    m.def("mttkrp3_tiles", [](py::dict part, int mode, arr<double> A, arr<double> B,
                              arr<double> C, int R, py::sequence dims) {
        size_t d[3];
        dims_from(dims, d);
        Partition3 p = part_from_dict(part);
        std::vector<double> out(d[mode] * size_t(R), 0.0);
        mttkrp3_tiles(p, mode, A.data(), B.data(), C.data(), R, d, out.data());
        return np(out);
    });

    m.def("gram", [](arr<double> F, int R) {
        const size_t rows = F.size() / size_t(R);
        std::vector<double> G(size_t(R) * R);
        gram(F.data(), rows, R, G.data());
        return np(G);
    });

    m.def("pinv_sym", [](arr<double> A, int R) {
        std::vector<double> out(size_t(R) * R);
        const int sweeps = pinv_sym(A.data(), R, out.data());
        return py::make_tuple(np(out), sweeps);
    });


    // ---------------- generic N-order ----------------
    m.def("reorder_nd", [](arr<uint32_t> coords, arr<double> vals, py::sequence dims,
                           const std::string& how, int rounds, size_t sample_budget) {
        CooN t = coon_from(coords, vals, dims);
        std::vector<std::vector<uint32_t>> rank;
        reorder_nd(t, how, rounds, sample_budget, rank);
        py::list rl;
        for (auto& r : rank) rl.append(np(r));
        return py::make_tuple(coords_np(t), rl);
    });
    m.def("splitbit_hash", &splitbit_hash);
    m.def(
        "dense_nd",
        [](arr<uint32_t> coords, arr<double> vals, py::sequence dims, double thr,
           std::array<int, 3> inner) {
            CooN t = coon_from(coords, vals, dims);
            UnitsN u;
            dense_nd(t, thr, inner.data(), u);
            return units_to_dict(u);
        },
        py::arg("coords"), py::arg("vals"), py::arg("dims"), py::arg("thr"),
        py::arg("inner") = std::array<int, 3>{0, 1, 2});
    m.def(
        "views_nd",
        [](arr<uint32_t> coords, arr<double> vals, py::sequence dims, py::object is_dense,
           bool enabled, std::array<int, 3> inner) {
            CooN t = coon_from(coords, vals, dims);
            std::vector<uint8_t> isd;
            if (!is_dense.is_none()) isd = vec(is_dense.cast<arr<uint8_t>>());
            unsigned mask = 0;
            if (enabled)
                for (int x : inner) mask |= 1u << x;
            ViewN v;
            views_nd(t, isd, mask, v);
            return viewn_to_list(v);
        },
        py::arg("coords"), py::arg("vals"), py::arg("dims"), py::arg("is_dense"),
        py::arg("enabled"), py::arg("inner") = std::array<int, 3>{0, 1, 2});
    m.def("mttkrp_seg_nd", [](arr<uint32_t> coords, arr<double> vals, py::sequence dims,
                              py::list views, int n, bool use_skip, py::list F, int R,
                              py::object init) {
        CooN t = coon_from(coords, vals, dims);
        ViewN v = viewn_from_list(views);
        std::vector<double> out(t.dims[n] * size_t(R), 0.0);
        if (!init.is_none()) out = vec(init.cast<arr<double>>());
        mttkrp_seg_nd(t, v, n, use_skip, flist(F), R, out.data());
        return np(out);
    });
    m.def("mttkrp_units_nd", [](arr<uint32_t> coords, arr<double> vals, py::sequence dims,
                                py::dict units, int n, py::list F, int R) {
        CooN t = coon_from(coords, vals, dims);
        UnitsN u = units_from_dict(units, t.N);
        std::vector<double> out(t.dims[n] * size_t(R), 0.0);
        mttkrp_units_nd(t, u, n, flist(F), R, out.data());
        return np(out);
    });
    m.def("chol_solve_nd", [](arr<double> FtF, arr<double> FtV, int R) {
        const size_t dim = FtV.size() / size_t(R);
        std::vector<double> out(dim * size_t(R));
        chol_solve_nd(FtF.data(), FtV.data(), out.data(), dim, R);
        return np(out);
    });
    m.def("als_nd", [](arr<uint32_t> coords, arr<double> vals, py::sequence dims, py::list rank,
                       int R, unsigned seed, bool svd, bool dense, double thr, int iters,
                       std::array<int, 3> inner) {
        CooN t = coon_from(coords, vals, dims);
        std::vector<std::vector<uint32_t>> rk;
        for (auto r : rank) rk.push_back(vec(r.cast<arr<uint32_t>>()));
        AlsNOpts o;
        o.R = R;
        o.seed = seed;
        o.svd = svd;
        o.dense = dense;
        o.threshold = thr;
        for (int x = 0; x < 3; ++x) o.inner[x] = inner[x];
        AlsNState st;
        {
            py::gil_scoped_release rel;
            als_nd(t, rk, o, iters, st);
        }
        return py::make_tuple(np(st.fits), np(st.iprod), np(st.model2), flist_np(st.F),
                              np(st.lambda));
    }, py::arg("coords"), py::arg("vals"), py::arg("dims"), py::arg("rank"), py::arg("R"),
       py::arg("seed"), py::arg("svd"), py::arg("dense"), py::arg("thr"), py::arg("iters"),
       py::arg("inner") = std::array<int, 3>{0, 1, 2});
    // als_nd's fits and per-iteration wall times (ms): the generic CPU baseline
    m.def("als_nd_timed", [](arr<uint32_t> coords, arr<double> vals, py::sequence dims,
                             py::list rank, int R, unsigned seed, double thr, int iters) {
        CooN t = coon_from(coords, vals, dims);
        std::vector<std::vector<uint32_t>> rk;
        for (auto r : rank) rk.push_back(vec(r.cast<arr<uint32_t>>()));
        AlsNOpts o;
        o.R = R;
        o.seed = seed;
        o.dense = true;
        o.threshold = thr;
        AlsNState st;
        {
            py::gil_scoped_release rel;
            als_nd(t, rk, o, iters, st);
        }
        return py::make_tuple(np(st.fits), np(st.ms));
    });
    m.def("residual_nd", [](arr<uint32_t> coords, arr<double> vals, py::sequence dims, py::list F,
                            arr<double> lam, int R) {
        CooN t = coon_from(coords, vals, dims);
        return residual_nd(t, flist(F), vec(lam), R);
    });
    m.def("selftest_tensor", []() {
        CooN t;
        std::vector<std::vector<double>> F;
        selftest_tensor(t, F);
        return py::make_tuple(coords_np(t), np(t.val),
                              py::make_tuple(t.dims[0], t.dims[1], t.dims[2], t.dims[3]),
                              flist_np(F));
    });

    m.def("sgd3_sample", [](uint64_t seed, uint32_t batch, uint64_t nnz) {
        return np(sgd3_sample(seed, batch, nnz));
    });
    // one SGD step over `idx` on copies of the factors; returns (A, B, C)
    m.def("sgd3_step", [](arr<uint64_t> coords, arr<double> vals, arr<uint32_t> idx,
                          arr<double> A, arr<double> B, arr<double> C, arr<double> lam, int R,
                          double gamma) {
        std::vector<double> a = vec(A), b = vec(B), c = vec(C);
        sgd3_step(vec(coords), vec(vals), vec(idx), a.data(), b.data(), c.data(), lam.data(), R,
                  gamma);
        return py::make_tuple(np(a), np(b), np(c));
    });
    m.def("sgd3_normalize", [](arr<double> F, size_t rows, int R) {
        std::vector<double> f = vec(F), lam(static_cast<size_t>(R));
        sgd3_normalize(f.data(), rows, R, lam.data());
        return py::make_tuple(np(f), np(lam));
    });
    m.def("sgd3_loss", [](arr<uint64_t> coords, arr<double> vals, arr<uint32_t> idx,
                          arr<double> A, arr<double> B, arr<double> C, arr<double> lam, int R) {
        return sgd3_loss(vec(coords), vec(vals), vec(idx), A.data(), B.data(), C.data(),
                         lam.data(), R);
    });

    py::class_<PyAls3>(m, "Als3")
        .def(py::init([](py::list residual, py::object dense_view, py::object tiles, double x_sq,
                         py::sequence dims, int R, arr<double> A, arr<double> B, arr<double> C,
                         py::object lam) {
            auto* s = new PyAls3();
            s->residual = view_from_list(residual);
            if (!dense_view.is_none())
            {
                s->dense_view = view_from_list(dense_view.cast<py::list>());
                s->has_dv = true;
            }
            if (!tiles.is_none())
            {
                s->tiles = part_from_dict(tiles.cast<py::dict>());
                s->has_tiles = !s->tiles.tiles.empty();
            }
            s->x_sq = x_sq;
            s->st.R = R;
            dims_from(dims, s->st.dims);
            s->st.F[0] = vec(A);
            s->st.F[1] = vec(B);
            s->st.F[2] = vec(C);
            if (lam.is_none())
                s->st.lambda.assign(size_t(R), 1.0);
            else
                s->st.lambda = vec(lam.cast<arr<double>>());
            return s;
        }))
        .def("iterate",
             [](PyAls3& s, int iters) {
                 std::vector<double> f(iters), ms(iters), mm(iters);
                 Als3Input in = s.input();
                 {
                     py::gil_scoped_release rel;
                     als3_iterate(in, s.st, iters, f.data(), ms.data(), mm.data());
                 }
                 return py::make_tuple(np(f), np(ms), np(mm));
             })
        .def("factor", [](PyAls3& s, int m) { return np(s.st.F[m]); })
        .def("lam", [](PyAls3& s) { return np(s.st.lambda); })
        .def("residual", [](PyAls3& s, bool with_lambda) {
            double r = 0, x = 0;
            residual3(s.input(), s.st, with_lambda, &r, &x);
            return py::make_tuple(r, x);
        });
}
