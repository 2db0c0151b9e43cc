// NTT kernels for gfx950 and the NttEngine that plans and launches them.
//
// One templated pass kernel covers every case: a workgroup owns a tile of
// 2^LB words = 2^LT transform points x 2^LI independent lines, held as 16
// words per thread. "ROW" tiles hold 2^LI contiguous rows (transform index in
// the low tile bits); "COL" tiles hold 2^LI adjacent columns of stride 2^l2
// (transform index in the high tile bits). The LT transform bits are
// butterflied four at a time in registers (radix-16 windows, high->low for the
// Cooley-Tukey forward, low->high for the Gentleman-Sande inverse) with LDS
// exchanges between windows. Twiddles come from one table per domain indexed by
// (n + j) >> (b + 1); see ntt_engine.hpp for the formulation.
//
// Arithmetic: Shoup multiplication a*w - hi(a*w')*q with w' = floor(w 2^k / q)
// (V. Shoup; D. Harvey, "Faster arithmetic for number-theoretic transforms",
// J. Symb. Comp. 2014): result in [0, 2q) for any word a. With 4q below the
// word size ("lazy"), forward values live in [0, 4q) and inverse values in
// [0, 2q); otherwise every butterfly keeps [0, 2q). Outputs are canonical.
// A Barrett variant (`-barrett`, moduli below 2^(k-2)) keeps canonical values
// and multiplies by bare twiddles with one constant per modulus (see
// ntt_kernels.hpp), so its tables hold one word per entry instead of a pair.
#include <hip/hip_runtime.h>

#include "json.hpp"
#include "ntt_kernels.hpp"
#include "planner.hpp"

#include <algorithm>

namespace cbw {
namespace ntt_detail {

template <>
std::map<PassKey, PassLaunch<std::uint32_t>>& registry<std::uint32_t>() {
    static std::map<PassKey, PassLaunch<std::uint32_t>> table;
    return table;
}
template <>
std::map<PassKey, PassLaunch<std::uint64_t>>& registry<std::uint64_t>() {
    static std::map<PassKey, PassLaunch<std::uint64_t>> table;
    return table;
}

}  // namespace ntt_detail

namespace {
using namespace ntt_detail;

void ensure_registered() {
    static const bool once = [] {
        register_u32_lazy();
        register_u32_strict();
        register_u64_lazy();
        register_u64_strict();
        register_u32_barrett();
        register_u64_barrett();
        register_alt_u32();
        register_alt_u64();
        return true;
    }();
    (void)once;
}

template <class W>
PassLaunch<W> find_pass(const PassKey& key) {
    ensure_registered();
    auto it = registry<W>().find(key);
    if (it == registry<W>().end()) throw NotSupported("NTT pass shape has no gfx950 kernel");
    return it->second;
}

// ---- host tables ------------------------------------------------------------

template <class W>
W shoup_factor(std::uint64_t w, std::uint64_t q) {
    const unsigned bits = sizeof(W) * 8;
    return static_cast<W>((static_cast<u128>(w) << bits) / q);
}

// Forward table T[k] (k = m + i, m = 2^s): negacyclic psi^bitrev_logn(k);
// cyclic w^(bitrev_s(i) n / 2m). The inverse table uses the inverse root.
template <class W>
std::vector<TwPair<W>> make_table(std::uint32_t log_n, std::uint64_t q, std::uint64_t root, bool negacyclic) {
    const std::uint64_t n = std::uint64_t{1} << log_n;
    std::vector<TwPair<W>> table(n);
    table[0] = {W(1), shoup_factor<W>(1, q)};
    if (negacyclic) {
        // powers[e] = root^e for e < n, then scatter by bit reversal.
        std::uint64_t p = 1;
        for (std::uint64_t e = 0; e < n; ++e) {
            const std::uint64_t k = bit_reverse(e, log_n);
            if (k) table[k] = {W(p), shoup_factor<W>(p, q)};
            p = mulmod(p, root, q);
        }
    } else {
        std::vector<std::uint64_t> pw(n / 2);
        std::uint64_t p = 1;
        for (std::uint64_t e = 0; e < n / 2; ++e, p = mulmod(p, root, q)) pw[e] = p;
        for (std::uint32_t s = 0; s < log_n; ++s) {
            const std::uint64_t m = std::uint64_t{1} << s;
            for (std::uint64_t i = 0; i < m; ++i) {
                const std::uint64_t e = bit_reverse(i, s) * (n / (2 * m));
                table[m + i] = {W(pw[e]), shoup_factor<W>(pw[e], q)};
            }
        }
    }
    return table;
}

template <class W>
struct EngineImplT {
    NttEngineConfig cfg;
    bool lazy = false;
    int arith = kStrict;
    std::uint32_t l1 = 0, l2 = 0;
    DeviceBuffer tables, domains, poly_domain, in_off, out_off;
    struct Launch {
        PassLaunch<W> fn;
        unsigned grid;
        PassArgs<W> args;
        bool reads_workspace, writes_workspace;
        int lt, prefix_bits;
        bool last;
    };
    std::vector<Launch> launches;
    std::string json_shape;

    explicit EngineImplT(const NttEngineConfig& c) : cfg(c) {
        const std::uint32_t log_n = c.log_n;
        const std::uint64_t n = std::uint64_t{1} << log_n;
        const unsigned bits = sizeof(W) * 8;
        std::uint64_t max_q = 0;
        for (const auto& d : c.domains) max_q = std::max(max_q, d.modulus);
        lazy = !c.force_strict && !c.barrett && max_q < (std::uint64_t{1} << (bits - 2));
        supported(!c.barrett || max_q < (std::uint64_t{1} << (bits - 2)),
                  "Barrett arithmetic needs every modulus below 2^" + std::to_string(bits - 2));
        arith = c.barrett ? kBarrett : lazy ? kLazy : kStrict;
        const std::uint64_t polys = c.polynomials.empty() ? c.batch : c.polynomials.size();
        require(polys >= 1 && polys <= 0xffffffffull, "NTT batch must be in [1, 2^32)");
        const bool offsets = !c.polynomials.empty();
        if (offsets) {
            std::vector<std::uint32_t> pd;
            std::vector<std::uint64_t> io, oo;
            for (const auto& p : c.polynomials) {
                pd.push_back(p.domain);
                io.push_back(p.input_offset);
                oo.push_back(p.output_offset);
            }
            poly_domain.upload(pd);
            in_off.upload(io);
            out_off.upload(oo);
        }
        const bool mixed = c.domains.size() > 1;
        PassArgs<W> base{};
        base.polys = static_cast<std::uint32_t>(polys);
        constexpr int LB = kTileLog;
        const bool ct = !c.inverse;
        // Which physical boundaries differ from the algorithm's native order
        // (forward: natural in / bit-reversed out; inverse: the opposite).
        const bool perm_in = ct ? c.input_bit_reversed : !c.input_bit_reversed;
        const bool perm_out = ct ? !c.output_bit_reversed : c.output_bit_reversed;
        if (log_n <= 12) {
            // One pass: whole polynomials per workgroup (one per tile if
            // domains mix or polynomials sit at explicit offsets).
            const int li = LB - int(log_n);
            supported((!mixed && !offsets) || li == 0, "mixed-domain or offset batches need log n >= 12");
            l1 = 0;
            l2 = log_n;
            const std::uint64_t per_tile = std::uint64_t{1} << li;
            const std::uint64_t tiles = (polys + per_tile - 1) / per_tile;
            Launch L{};
            L.fn = find_pass<W>(PassKey{arith, int(log_n), int(log_n), li, false, ct, perm_in, perm_out, true});
            L.grid = unsigned(tiles);
            L.args = base;
            L.args.tiles = unsigned(tiles);
            L.args.in_off = in_off.as<std::uint64_t>();
            L.args.out_off = out_off.as<std::uint64_t>();
            L.args.reduce_input = c.reduce_input;
            L.lt = int(log_n);
            L.prefix_bits = 0;
            L.last = true;
            launches.push_back(L);
            json_shape = "{\"passes\":1,\"tile_log\":" + std::to_string(LB) + "}";
        } else {
            supported(log_n <= 20, "NTT lengths above 2^20 are not yet lowered for gfx950");
            l1 = std::uint32_t(split_l1(int(log_n)));
            if (c.split_high && c.split_high != l1) {
                supported(alt_split(int(log_n), int(c.split_high)), "NTT split has no gfx950 kernels");
                l1 = c.split_high;
            }
            l2 = log_n - l1;
            const int col_li = c.wide_columns ? kWideColLines : kColLines;
            const int rli = row_lines(int(l1), int(l2));
            const std::uint64_t col_tiles = polys << (l2 - col_li);
            const std::uint64_t row_tiles = polys << (l1 - rli);
            require(col_tiles <= 0xffffffffull && row_tiles <= 0xffffffffull, "NTT batch exceeds the grid");
            Launch A{}, B{};
            // Pass A: high bits (columns); pass B: low bits (rows).
            A.args = base;
            A.args.tiles = unsigned(col_tiles);
            A.grid = unsigned(col_tiles);
            A.lt = int(l1);
            A.prefix_bits = 0;
            A.last = !ct;
            B.args = base;
            B.args.tiles = unsigned(row_tiles);
            B.grid = unsigned(row_tiles);
            B.lt = int(l2);
            B.prefix_bits = int(l1);
            B.last = ct;
            A.fn = find_pass<W>(
                PassKey{arith, int(log_n), int(l1), col_li, true, ct, ct && perm_in, !ct && perm_out, false});
            B.fn = find_pass<W>(
                PassKey{arith, int(log_n), int(l2), rli, false, ct, !ct && perm_in, ct && perm_out, false});
            if (ct) {  // forward: A reads the input, B writes the output
                A.args.in_off = in_off.as<std::uint64_t>();
                A.args.reduce_input = c.reduce_input;
                A.writes_workspace = true;
                B.reads_workspace = true;
                B.args.out_off = out_off.as<std::uint64_t>();
                launches = {A, B};
            } else {  // inverse: B reads the input, A writes the output
                B.args.in_off = in_off.as<std::uint64_t>();
                B.args.reduce_input = c.reduce_input;
                B.writes_workspace = true;
                A.reads_workspace = true;
                A.args.out_off = out_off.as<std::uint64_t>();
                launches = {B, A};
            }
            json_shape = "{\"passes\":2,\"high_bits\":" + std::to_string(l1) + ",\"low_bits\":" +
                         std::to_string(l2) + ",\"column_tile_lines\":" + std::to_string(1 << col_li) +
                         ",\"row_tile_lines\":" + std::to_string(1 << rli) + "}";
        }
        // Device domain records and their twiddle chunks (one layout for all
        // domains, so the phase offsets are shared).
        if (arith == kBarrett) build_tables<W>(c, n, ct);
        else build_tables<TwPair<W>>(c, n, ct);
    }

    // Entry E: a Shoup pair, or the bare twiddle word (Barrett).
    template <class E>
    void build_tables(const NttEngineConfig& c, std::uint64_t n, bool ct) {
        std::vector<DeviceDomain<W>> host_domains;
        std::vector<E> all_tables;
        for (const auto& d : c.domains) {
            const std::uint64_t q = d.modulus;
            const std::uint64_t root = c.inverse ? invmod(d.root, q) : d.root;
            const auto pairs = make_table<W>(c.log_n, q, root, c.negacyclic);
            DeviceDomain<W> dd{};
            dd.q = W(q);
            dd.q2 = W(2 * q);
            dd.nq = W(0) - W(q);
            dd.rwp = shoup_factor<W>(1, q);
            const std::uint64_t ninv = invmod(n % q, q);
            dd.ninv = {W(ninv), shoup_factor<W>(ninv, q)};
            const std::uint64_t last = mulmod(pairs[1].w, ninv, q);
            dd.last = {W(last), shoup_factor<W>(last, q)};
            unsigned qbits = 0;
            while (qbits < 64 && (q >> qbits) != 0) ++qbits;
            dd.qbits = qbits;
            // mu = floor(2^(2b+1) / q) < 2^(b+2) fits the word for q < 2^(k-2).
            dd.mu = qbits + 2 <= sizeof(W) * 8 ? W((u128{1} << (2 * qbits + 1)) / q) : W(0);
            std::vector<E> table(pairs.size());
            for (std::size_t k = 0; k < pairs.size(); ++k) {
                if constexpr (std::is_same_v<E, W>) {
                    table[k] = pairs[k].w;
                } else {
                    table[k] = pairs[k];
                    if (ct && lazy) table[k].w = W(0) - table[k].w;  // lazy Cooley-Tukey butterflies take -w
                }
            }
            dd.tw = all_tables.size();
            for (auto& L : launches)
                append_pass_chunks<E>(all_tables, std::size_t(dd.tw), table, L.lt, L.prefix_bits, ct, L.last,
                                      L.args.phase_off);
            host_domains.push_back(dd);
        }
        require(all_tables.size() * sizeof(E) < 0x7fffffffull, "NTT twiddle tables exceed 2 GiB");
        tables.upload(all_tables);
        domains.upload(host_domains);
        const std::size_t per_domain = all_tables.size() / c.domains.size();
        for (auto& L : launches) {
            L.args.tw_bytes = static_cast<std::uint32_t>(per_domain * sizeof(E));
            L.args.domains = domains.as<DeviceDomain<W>>();
            L.args.tw = tables.as<E>();
            L.args.poly_domain = poly_domain.as<std::uint32_t>();
        }
    }

    std::size_t workspace_bytes() const {
        if (launches.size() < 2) return 0;
        const std::uint64_t polys = cfg.polynomials.empty() ? cfg.batch : cfg.polynomials.size();
        return static_cast<std::size_t>((polys << cfg.log_n) * sizeof(W));
    }

    void execute(const void* in, void* out, void* ws, hipStream_t stream) const {
        require(launches.size() < 2 || ws != nullptr, "two-pass NTT needs a workspace");
        for (const auto& L : launches) {
            PassArgs<W> a = L.args;
            a.in = static_cast<const W*>(L.reads_workspace ? ws : in);
            a.out = static_cast<W*>(L.writes_workspace ? ws : out);
            L.fn(a, L.grid, stream);
            hip_check(hipGetLastError(), "NTT pass launch");
        }
    }
};

}  // namespace

struct NttEngine::Impl {
    std::unique_ptr<EngineImplT<std::uint32_t>> u32;
    std::unique_ptr<EngineImplT<std::uint64_t>> u64;
};

NttEngine::NttEngine(const NttEngineConfig& c) : impl_(new Impl) {
    require(c.word_bits == 32 || c.word_bits == 64, "NTT word bits must be 32 or 64");
    require(c.log_n >= 1 && c.log_n <= 30, "NTT log n must be in [1, 30]");
    require(!c.domains.empty(), "NTT needs at least one domain");
    for (const auto& d : c.domains) {
        require(d.modulus >= 3 && (c.word_bits == 64 ? d.modulus < (1ull << 63) : d.modulus < (1ull << 31)),
                "NTT modulus out of range for the word size");
        require(d.root != 0 && d.root < d.modulus, "NTT root must be in [1, q)");
    }
    for (const auto& p : c.polynomials) require(p.domain < c.domains.size(), "polynomial domain out of range");
    if (c.word_bits == 32)
        impl_->u32 = std::make_unique<EngineImplT<std::uint32_t>>(c);
    else
        impl_->u64 = std::make_unique<EngineImplT<std::uint64_t>>(c);
    const bool two = passes() == 2;
    const bool other_split = two && c.split_high && c.split_high != std::uint32_t(split_l1(int(c.log_n)));
    algorithm_ = std::string("ntt-u") + std::to_string(c.word_bits) + (c.negacyclic ? "-negacyclic" : "-cyclic") +
                 (two ? "-two-pass-r16" : "-resident-r16") + (c.force_strict ? "-strict" : "") +
                 (c.barrett ? "-barrett" : "") +
                 (two && c.wide_columns ? "-c32" : "") +
                 (other_split ? "-h" + std::to_string(c.split_high) : "");
    json::Writer w;
    w.begin_object()
        .field("schema_version", 1u)
        .field("operator", "ntt")
        .field("algorithm", algorithm_)
        .field("word_bits", c.word_bits)
        .field("log_n", c.log_n)
        .field("ring", c.negacyclic ? "negacyclic" : "cyclic")
        .field("direction", c.inverse ? "inverse" : "forward")
        .field("input_order", c.input_bit_reversed ? "bit_reversed" : "natural")
        .field("output_order", c.output_bit_reversed ? "bit_reversed" : "natural")
        .field("arithmetic", c.barrett ? "barrett" : "shoup")
        .field("lazy_reduction", impl_->u32 ? impl_->u32->lazy : impl_->u64->lazy)
        .key("shape")
        .value_raw(impl_->u32 ? impl_->u32->json_shape : impl_->u64->json_shape)
        .field("workspace_bytes", std::uint64_t(workspace_bytes()))
        .end_object();
    mapping_json_ = w.str();
}

NttEngine::~NttEngine() = default;

std::vector<std::uint32_t> ntt_other_splits(std::uint32_t log_n) {
    std::vector<std::uint32_t> out;
    if (log_n < 13 || log_n > 20) return out;
    const int l1 = split_l1(int(log_n));
    for (const int h : {l1 - 1, l1 + 1})
        if (alt_split(int(log_n), h)) out.push_back(std::uint32_t(h));
    return out;
}

std::size_t NttEngine::workspace_bytes() const {
    return impl_->u32 ? impl_->u32->workspace_bytes() : impl_->u64->workspace_bytes();
}

std::uint32_t NttEngine::passes() const {
    return std::uint32_t(impl_->u32 ? impl_->u32->launches.size() : impl_->u64->launches.size());
}

void NttEngine::execute(const void* in, void* out, void* ws, hipStream_t stream) const {
    if (impl_->u32)
        impl_->u32->execute(in, out, ws, stream);
    else
        impl_->u64->execute(in, out, ws, stream);
}

// ---- cubutterfly.h NTT plans -------------------------------------------------

namespace {

std::string join(const std::vector<std::string>& names) {
    std::string out;
    for (const auto& n : names) out += (out.empty() ? "" : ", ") + n;
    return out;
}

// 32-column tiles are the static choice where they measured faster: u32
// 2^16-point transforms (C2 step 43.9-44.7 us against 44.9-45.3 us).
bool wide_columns_default(const Request& r) { return r.word_bits == 32 && r.log_n == 16; }

std::vector<std::uint32_t> other_splits(const Request& r) { return ntt_other_splits(r.log_n); }

// Name of the static model's lowering: resident up to 2^12, then two passes.
std::string default_name(const Request& r) {
    return "ntt-u" + std::to_string(r.word_bits) + (r.negacyclic ? "-negacyclic" : "-cyclic") +
           (r.log_n <= 12 ? "-resident-r16" : "-two-pass-r16");
}

class NttExecutor final : public Executor {
  public:
    explicit NttExecutor(const Request& r) {
        NttEngineConfig c;
        c.word_bits = r.word_bits;
        c.log_n = r.log_n;
        c.negacyclic = r.negacyclic;
        c.inverse = r.inverse;
        c.input_bit_reversed = r.input_bit_reversed;
        c.output_bit_reversed = r.output_bit_reversed;
        c.reduce_input = true;  // reference_ntt reduces inputs mod q (src/reference.cpp:601-603)
        c.batch = r.batch;
        // Root conventions of the reference (src/reference.cpp:564-582;
        // crypto_ntt_bench.cu:273-323).
        const std::uint64_t w = primitive_root_pow2(r.log_n, r.modulus);
        std::uint64_t root = w;
        if (r.negacyclic) {
            if (r.psi) {
                const std::uint64_t order = std::uint64_t{2} << r.log_n;
                require(r.psi < r.modulus && powmod(r.psi, order >> 1, r.modulus) == r.modulus - 1,
                        "psi must be a primitive 2n-th root of unity");
                root = r.psi;
            } else {
                root = psi_for_root(r.log_n, r.modulus, w);
            }
        }
        c.domains.push_back({r.modulus, root});
        if (r.pitched) {  // rows a pitch apart: one polynomial per tile at its own offset
            require(r.batch <= 0xffffffffull, "NTT batch must be below 2^32");
            c.polynomials.reserve(r.batch);
            for (std::uint64_t b = 0; b < r.batch; ++b)
                c.polynomials.push_back({0u, b * r.in_batch_stride, b * r.out_batch_stride});
        }
        const std::string suffix = r.pitched ? "-pitched" : "";
        const std::vector<std::string> names = ntt_candidates(r);
        supported(r.variant.empty() || std::find(names.begin(), names.end(), r.variant) != names.end(),
                  "'" + r.variant + "' is not a lowering of this NTT (available: " + join(names) + ")");
        c.force_strict = r.variant == default_name(r) + "-strict" + suffix;
        c.barrett = r.variant == default_name(r) + "-barrett" + suffix;
        c.wide_columns = r.variant.empty() ? wide_columns_default(r) : r.variant == default_name(r) + "-c32" + suffix;
        for (const std::uint32_t h : other_splits(r))
            if (r.variant == default_name(r) + "-h" + std::to_string(h) + suffix) c.split_high = h;
        engine_ = std::make_unique<NttEngine>(c);
        algorithm = engine_->algorithm() + (r.pitched ? "-pitched" : "");
        mapping_json = engine_->mapping_json();
        reason = engine_->passes() == 1
                     ? "whole polynomials resident in one workgroup (radix-16 register windows, LDS exchange)"
                     : "two passes over high/low index bits (coalesced column and row tiles), merged-twist "
                       "Cooley-Tukey / Gentleman-Sande with Shoup arithmetic";
        if (c.barrett) reason += "; Barrett products (one constant per modulus, single-word twiddle tables)";
    }
    std::size_t workspace_bytes() const override { return engine_->workspace_bytes(); }
    void execute(const void* in, void* out, void* ws, hipStream_t stream) override {
        engine_->execute(in, out, ws, stream);
    }

  private:
    std::unique_ptr<NttEngine> engine_;
};

}  // namespace

std::unique_ptr<Executor> make_ntt_executor(const Request& r) { return std::make_unique<NttExecutor>(r); }

// Lazy reduction (values in [0, 2q) / [0, 4q) between stages) where the
// modulus leaves two spare bits, and the fully reduced butterflies.
// Two-pass transforms also offer 32-column tiles in the column pass (`-c32`:
// 128 / 256-byte row segments instead of 64 / 128) and, at 2^15..2^17, the
// neighbouring splits of the high and low bits (`-h<l1>`).
std::vector<std::string> ntt_candidates(const Request& r) {
    const std::string suffix = r.pitched ? "-pitched" : "";
    std::vector<std::string> names{default_name(r) + suffix};
    if (r.modulus < (std::uint64_t{1} << (r.word_bits - 2))) names.push_back(default_name(r) + "-strict" + suffix);
    if (r.log_n >= 13 && r.log_n <= 20) {
        names.push_back(default_name(r) + "-c32" + suffix);
        if (wide_columns_default(r)) std::rotate(names.begin(), names.end() - 1, names.end());  // the default first
    }
    for (const std::uint32_t h : other_splits(r)) names.push_back(default_name(r) + "-h" + std::to_string(h) + suffix);
    if (r.modulus < (std::uint64_t{1} << (r.word_bits - 2))) names.push_back(default_name(r) + "-barrett" + suffix);
    return names;
}

}  // namespace cbw
