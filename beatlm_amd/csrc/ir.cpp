// C++ restatement of the reference core's kernel IR, lowering, splitting and
// memory planner for the ViT encoder block's operations, behind the C API of
// include/beatlm_ir.h. Each function cites what it restates in
// crates/beatlm-core/src/{kernel,memory,device}.rs.
#include "../../include/beatlm_ir.h"

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <set>
#include <string>
#include <vector>

namespace {

thread_local std::string g_error;

int err(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
    return code;
}

// kernel.rs:381: kernels index with 32-bit integers.
constexpr uint64_t MAX_ELEMENTS = 0x7fffffffULL;
// The reference's tiles (kernel.rs:396-414): 64 rows; 64 or 32 columns.
constexpr uint32_t TILE_ROWS = 64;
constexpr uint32_t NARROW_COLUMNS = 32;
constexpr uint32_t LAYER_NORM_LANES = 64, SOFTMAX_LANES = 256, ELEMENT_GROUP = 256;

uint64_t product(std::initializer_list<uint64_t> dims) {
    uint64_t acc = 1;
    for (uint64_t d : dims) {
        if (d && acc > UINT64_MAX / d) return UINT64_MAX;
        acc *= d;
    }
    return acc;
}

bool role_whole_program(uint32_t r) { return r != BLI_ACTIVATION; }  // kernel.rs:437-440
bool role_written_by_op(uint32_t r) { return r == BLI_ACTIVATION || r == BLI_OUTPUT; }

struct TensorInfo {
    uint32_t role;
    uint64_t elements;
};

// ---- OpKind (kernel.rs:818-1131) ----

bool is_elementwise(uint32_t k) { return k >= BLI_OP_ADD; }

// Every tensor the operation reads with its element count (OpKind::reads, kernel.rs:924-975).
std::vector<std::pair<uint32_t, uint64_t>> op_reads(const bli_op &o) {
    const uint32_t *t = o.t, *d = o.d;
    std::vector<std::pair<uint32_t, uint64_t>> r;
    switch (o.kind) {
    case BLI_OP_LAYER_NORM: r = {{t[0], product({d[0], d[1]})}, {t[1], d[1]}, {t[2], d[1]}}; break;
    case BLI_OP_MATMUL:
        r = {{t[0], product({d[0], d[1]})}, {t[1], product({d[1], d[2]})}};
        if (t[2] != BLI_NONE) r.push_back({t[2], d[2]});
        break;
    case BLI_OP_PATCH_EMBED:
        r = {{t[0], product({d[0], d[2], d[1], d[2], d[3]})}, {t[1], product({d[2], d[2], d[3], d[4]})}};
        if (t[2] != BLI_NONE) r.push_back({t[2], d[4]});
        break;
    case BLI_OP_PREPEND_TOKEN: r = {{t[0], d[1]}, {t[1], product({d[0], d[1]})}}; break;
    case BLI_OP_TOKENS_TO_MAP: r = {{t[0], (product({d[0], d[1]}) + 1) * d[2]}}; break;
    case BLI_OP_ATTENTION_SCORES: r = {{t[0], product({d[0], 3, d[1], d[2]})}}; break;
    case BLI_OP_SOFTMAX: r = {{t[0], product({d[0], d[1]})}}; break;
    case BLI_OP_ATTENTION_VALUES:
        r = {{t[0], product({d[0], d[1], d[0]})}, {t[1], product({d[0], 3, d[1], d[2]})}};
        break;
    case BLI_OP_ADD: r = {{t[0], d[0]}, {t[1], d[0]}}; break;
    case BLI_OP_RELU:
    case BLI_OP_GELU:
    case BLI_OP_GELU_ERF:
    case BLI_OP_SCALE: r = {{t[0], d[0]}}; break;
    case BLI_OP_CHANNEL_SCALE: r = {{t[0], product({d[0], d[1]})}, {t[1], d[1]}}; break;
    case BLI_OP_CONV3X3:
        r = {{t[0], product({d[0], d[1], d[2]})}, {t[1], product({9, d[2], d[3]})}};
        if (t[2] != BLI_NONE) r.push_back({t[2], d[3]});
        break;
    case BLI_OP_CONV1X1:
        r = {{t[0], product({d[0], d[1], d[2]})}, {t[1], product({d[2], d[3]})}};
        if (t[2] != BLI_NONE) r.push_back({t[2], d[3]});
        break;
    case BLI_OP_CONV_TRANSPOSE:
        r = {{t[0], product({d[0], d[1], d[2]})}, {t[1], product({d[4], d[4], d[2], d[3]})}};
        if (t[2] != BLI_NONE) r.push_back({t[2], d[3]});
        break;
    case BLI_OP_RESIZE_BILINEAR: r = {{t[0], product({d[0], d[1], d[4]})}}; break;
    default: break;
    }
    return r;
}

// Conv2d3x3::out_height / strided (kernel.rs:479-507): a 3x3 window with
// padding 1 at `stride`, (extent - 1) / stride + 1.
uint32_t strided(uint32_t extent, uint32_t stride) { return (extent == 0 || stride == 0) ? 0 : (extent - 1) / stride + 1; }

// OpKind::output_elements (kernel.rs:977-1005).
uint64_t op_output(const bli_op &o) {
    const uint32_t *d = o.d;
    switch (o.kind) {
    case BLI_OP_LAYER_NORM: return product({d[0], d[1]});
    case BLI_OP_MATMUL: return product({d[0], d[2]});
    case BLI_OP_PATCH_EMBED: return product({d[0], d[1], d[4]});
    case BLI_OP_PREPEND_TOKEN: return ((uint64_t)d[0] + 1) * d[1];
    case BLI_OP_TOKENS_TO_MAP: return product({d[0], d[1], d[2]});
    case BLI_OP_ATTENTION_SCORES: return product({d[0], d[1], d[0]});
    case BLI_OP_SOFTMAX: return product({d[0], d[1]});
    case BLI_OP_ATTENTION_VALUES: return product({d[0], d[1], d[2]});
    case BLI_OP_ADD:
    case BLI_OP_RELU:
    case BLI_OP_GELU:
    case BLI_OP_GELU_ERF:
    case BLI_OP_SCALE: return d[0];
    case BLI_OP_CHANNEL_SCALE: return product({d[0], d[1]});
    case BLI_OP_CONV3X3: return product({strided(d[0], d[4]), strided(d[1], d[4]), d[3]});
    case BLI_OP_CONV1X1: return product({d[0], d[1], d[3]});
    case BLI_OP_CONV_TRANSPOSE: return product({d[0], d[4], d[1], d[4], d[3]});
    case BLI_OP_RESIZE_BILINEAR: return product({d[2], d[3], d[4]});
    default: return 0;
    }
}

// OpKind::has_zero_dimension (kernel.rs:1008-1046).
bool op_has_zero_dim(const bli_op &o) {
    const uint32_t *d = o.d;
    auto any0 = [&](int n) {
        for (int i = 0; i < n; i++)
            if (!d[i]) return true;
        return false;
    };
    switch (o.kind) {
    case BLI_OP_LAYER_NORM: case BLI_OP_SOFTMAX: case BLI_OP_PREPEND_TOKEN: case BLI_OP_CHANNEL_SCALE: return any0(2);
    case BLI_OP_MATMUL: case BLI_OP_ATTENTION_SCORES: case BLI_OP_ATTENTION_VALUES: case BLI_OP_TOKENS_TO_MAP: return any0(3);
    case BLI_OP_PATCH_EMBED: case BLI_OP_CONV3X3: case BLI_OP_CONV_TRANSPOSE: case BLI_OP_RESIZE_BILINEAR: return any0(5);
    case BLI_OP_CONV1X1: return any0(4);
    default: return any0(1);
    }
}

// ---- MainOp (kernel.rs:1393-1591) ----

struct MainOp {
    uint32_t kind = 0;                            // BL_MAIN_*
    uint32_t t[3] = {BLI_NONE, BLI_NONE, BLI_NONE};  // reads, in order
    uint32_t d[6] = {0, 0, 0, 0, 0, 0};
    float eps = 0.0f, scale = 1.0f;

    std::vector<uint32_t> reads() const {
        std::vector<uint32_t> r;
        for (uint32_t x : t)
            if (x != BLI_NONE) r.push_back(x);
        return r;
    }
    uint64_t output_elements() const {
        switch (kind) {
        case BL_MAIN_LAYER_NORM: case BL_MAIN_SOFTMAX: return product({d[0], d[1]});
        case BL_MAIN_MATMUL: return product({d[0], d[2]});
        case BL_MAIN_PATCH_EMBED: return product({d[0], d[1], d[4]});
        case BL_MAIN_PREPEND_TOKEN: return ((uint64_t)d[0] + 1) * d[1];
        case BL_MAIN_TOKENS_TO_MAP: return product({d[0], d[1], d[2]});
        case BL_MAIN_ATTENTION_SCORES: return product({d[0], d[1], d[0]});
        case BL_MAIN_ATTENTION_VALUES: case BL_MAIN_FLASH_ATTENTION: return product({d[0], d[1], d[2]});
        case BL_MAIN_MAP: return d[0];
        case BL_MAIN_CONV3X3: return product({strided(d[0], d[4]), strided(d[1], d[4]), d[3]});
        case BL_MAIN_CONV_TRANSPOSE: return product({d[0], d[4], d[1], d[4], d[3]});
        case BL_MAIN_RESIZE_BILINEAR: return product({d[2], d[3], d[4]});
        default: return 0;
        }
    }
    const char *name() const {  // MainOp::name (kernel.rs:1499-1515)
        switch (kind) {
        case BL_MAIN_CONV3X3: return "conv2d3x3";
        case BL_MAIN_CONV_TRANSPOSE: return "conv_transpose2d";
        case BL_MAIN_RESIZE_BILINEAR: return "resize_bilinear";
        case BL_MAIN_LAYER_NORM: return "layernorm";
        case BL_MAIN_MATMUL: return "matmul";
        case BL_MAIN_PATCH_EMBED: return "patch_embed";
        case BL_MAIN_PREPEND_TOKEN: return "prepend_token";
        case BL_MAIN_TOKENS_TO_MAP: return "tokens_to_map";
        case BL_MAIN_ATTENTION_SCORES: return "attention_scores";
        case BL_MAIN_SOFTMAX: return "softmax";
        case BL_MAIN_ATTENTION_VALUES: return "attention_values";
        case BL_MAIN_MAP: return "map";
        case BL_MAIN_FLASH_ATTENTION: return "flash_attention";
        default: return "?";
        }
    }
    // split_extent (kernel.rs:1521-1538)
    uint32_t split_extent() const {
        switch (kind) {
        case BL_MAIN_LAYER_NORM: case BL_MAIN_SOFTMAX: case BL_MAIN_MATMUL: return d[0];
        case BL_MAIN_PATCH_EMBED: return (uint32_t)std::min<uint64_t>(product({d[0], d[1]}), UINT32_MAX);
        case BL_MAIN_ATTENTION_SCORES: case BL_MAIN_ATTENTION_VALUES: case BL_MAIN_FLASH_ATTENTION: return d[0];
        case BL_MAIN_CONV3X3: return (uint32_t)std::min<uint64_t>(product({strided(d[0], d[4]), strided(d[1], d[4])}), UINT32_MAX);
        case BL_MAIN_CONV_TRANSPOSE: return (uint32_t)std::min<uint64_t>(product({d[0], d[4], d[1], d[4]}), UINT32_MAX);
        case BL_MAIN_RESIZE_BILINEAR: return (uint32_t)std::min<uint64_t>(product({d[2], d[3]}), UINT32_MAX);
        default: return (uint32_t)std::min<uint64_t>(output_elements(), UINT32_MAX);
        }
    }
    // The tiled kernel's output columns within a layer and its layers (kernel.rs:1575-1590).
    bool tile_columns_and_layers(uint32_t &cols, uint32_t &layers) const {
        switch (kind) {
        case BL_MAIN_MATMUL: cols = d[2]; layers = 1; return true;
        case BL_MAIN_PATCH_EMBED: cols = d[4]; layers = 1; return true;
        case BL_MAIN_ATTENTION_SCORES: cols = d[0]; layers = d[1]; return true;
        case BL_MAIN_ATTENTION_VALUES: cols = d[2]; layers = d[1]; return true;
        case BL_MAIN_CONV3X3: cols = d[3]; layers = 1; return true;
        default: return false;
        }
    }
    uint32_t tile_columns() const {  // tile(): narrow at <= 32 columns
        uint32_t c, l;
        if (!tile_columns_and_layers(c, l)) return 0;
        return c <= NARROW_COLUMNS ? 32 : 64;
    }
    // split_grain (kernel.rs:1541-1543); the flash kernel moves in 64 query rows.
    uint32_t split_grain() const {
        if (kind == BL_MAIN_FLASH_ATTENTION) return 64;
        return tile_columns() ? TILE_ROWS : 1;
    }
    uint64_t elements_per_unit() const {  // kernel.rs:1558-1571
        switch (kind) {
        case BL_MAIN_LAYER_NORM: case BL_MAIN_SOFTMAX: return d[1];
        case BL_MAIN_MATMUL: return d[2];
        case BL_MAIN_PATCH_EMBED: return d[4];
        case BL_MAIN_ATTENTION_SCORES: return product({d[1], d[0]});
        case BL_MAIN_ATTENTION_VALUES: case BL_MAIN_FLASH_ATTENTION: return product({d[1], d[2]});
        case BL_MAIN_CONV3X3: case BL_MAIN_CONV_TRANSPOSE: return d[3];
        case BL_MAIN_RESIZE_BILINEAR: return d[4];
        default: return 1;
        }
    }
    bool operator==(const MainOp &o) const {
        return kind == o.kind && !memcmp(t, o.t, sizeof t) && !memcmp(d, o.d, sizeof d) && eps == o.eps &&
               scale == o.scale;
    }
};

// Epilogue (kernel.rs:1593-1641).
struct Epi {
    uint32_t kind;          // BL_EPI_*
    uint32_t tensor = BLI_NONE;
    float factor = 0.0f;
    uint32_t channels = 0;
    bool operator==(const Epi &o) const {
        return kind == o.kind && tensor == o.tensor && factor == o.factor && channels == o.channels;
    }
};

const char *epi_name(uint32_t k) {
    switch (k) {
    case BL_EPI_ADD: return "add";
    case BL_EPI_RELU: return "relu";
    case BL_EPI_GELU: return "gelu";
    case BL_EPI_GELU_ERF: return "gelu_erf";
    case BL_EPI_SCALE: return "scale";
    case BL_EPI_CHANNEL_SCALE: return "channel_scale";
    default: return "?";
    }
}

// OpKind::standalone (kernel.rs:1049-1090).
void standalone(const bli_op &o, MainOp &m, std::vector<Epi> &e) {
    m = MainOp();
    e.clear();
    const uint32_t *t = o.t, *d = o.d;
    auto map = [&](uint32_t input, uint64_t elements) {
        m.kind = BL_MAIN_MAP;
        m.t[0] = input;
        m.d[0] = (uint32_t)std::min<uint64_t>(elements, UINT32_MAX);
    };
    switch (o.kind) {
    case BLI_OP_LAYER_NORM: m.kind = BL_MAIN_LAYER_NORM; m.t[0] = t[0]; m.t[1] = t[1]; m.t[2] = t[2]; m.d[0] = d[0]; m.d[1] = d[1]; m.eps = o.f; break;
    case BLI_OP_MATMUL:
        m.kind = BL_MAIN_MATMUL; m.t[0] = t[0]; m.t[1] = t[1]; m.t[2] = t[2];
        m.d[0] = d[0]; m.d[1] = d[1]; m.d[2] = d[2]; m.d[3] = t[2] != BLI_NONE;
        break;
    case BLI_OP_PATCH_EMBED:
        m.kind = BL_MAIN_PATCH_EMBED; m.t[0] = t[0]; m.t[1] = t[1]; m.t[2] = t[2];
        for (int i = 0; i < 5; i++) m.d[i] = d[i];
        m.d[5] = t[2] != BLI_NONE;
        break;
    case BLI_OP_PREPEND_TOKEN: m.kind = BL_MAIN_PREPEND_TOKEN; m.t[0] = t[0]; m.t[1] = t[1]; m.d[0] = d[0]; m.d[1] = d[1]; break;
    case BLI_OP_TOKENS_TO_MAP: m.kind = BL_MAIN_TOKENS_TO_MAP; m.t[0] = t[0]; m.d[0] = d[0]; m.d[1] = d[1]; m.d[2] = d[2]; break;
    case BLI_OP_ATTENTION_SCORES: m.kind = BL_MAIN_ATTENTION_SCORES; m.t[0] = t[0]; m.d[0] = d[0]; m.d[1] = d[1]; m.d[2] = d[2]; break;
    case BLI_OP_SOFTMAX: m.kind = BL_MAIN_SOFTMAX; m.t[0] = t[0]; m.d[0] = d[0]; m.d[1] = d[1]; break;
    case BLI_OP_ATTENTION_VALUES: m.kind = BL_MAIN_ATTENTION_VALUES; m.t[0] = t[0]; m.t[1] = t[1]; m.d[0] = d[0]; m.d[1] = d[1]; m.d[2] = d[2]; break;
    case BLI_OP_CONV3X3:
        m.kind = BL_MAIN_CONV3X3; m.t[0] = t[0]; m.t[1] = t[1]; m.t[2] = t[2];
        for (int i = 0; i < 5; i++) m.d[i] = d[i];
        m.d[5] = t[2] != BLI_NONE;
        break;
    case BLI_OP_CONV1X1:  // Conv2d1x1::as_matmul (kernel.rs:531-545): the [pixels][cin] image times [cin][cout]
        m.kind = BL_MAIN_MATMUL; m.t[0] = t[0]; m.t[1] = t[1]; m.t[2] = t[2];
        m.d[0] = (uint32_t)std::min<uint64_t>(product({d[0], d[1]}), UINT32_MAX); m.d[1] = d[2]; m.d[2] = d[3];
        m.d[3] = t[2] != BLI_NONE;
        break;
    case BLI_OP_CONV_TRANSPOSE:
        m.kind = BL_MAIN_CONV_TRANSPOSE; m.t[0] = t[0]; m.t[1] = t[1]; m.t[2] = t[2];
        for (int i = 0; i < 5; i++) m.d[i] = d[i];
        m.d[5] = t[2] != BLI_NONE;
        break;
    case BLI_OP_RESIZE_BILINEAR:
        m.kind = BL_MAIN_RESIZE_BILINEAR; m.t[0] = t[0];
        for (int i = 0; i < 5; i++) m.d[i] = d[i];
        break;
    case BLI_OP_ADD: map(t[0], d[0]); e.push_back({BL_EPI_ADD, t[1]}); break;
    case BLI_OP_RELU: map(t[0], d[0]); e.push_back({BL_EPI_RELU}); break;
    case BLI_OP_GELU: map(t[0], d[0]); e.push_back({BL_EPI_GELU}); break;
    case BLI_OP_GELU_ERF: map(t[0], d[0]); e.push_back({BL_EPI_GELU_ERF}); break;
    case BLI_OP_SCALE: map(t[0], d[0]); e.push_back({BL_EPI_SCALE, BLI_NONE, o.f}); break;
    case BLI_OP_CHANNEL_SCALE: map(t[0], product({d[0], d[1]})); e.push_back({BL_EPI_CHANNEL_SCALE, t[1], 0.0f, d[1]}); break;
    }
}

// OpKind::as_epilogue (kernel.rs:1094-1113): the step this op is when `chain` flows into it.
bool as_epilogue(const bli_op &o, uint32_t chain, Epi &step) {
    const uint32_t *t = o.t;
    switch (o.kind) {
    case BLI_OP_ADD:
        if (t[0] == chain && t[1] != chain) { step = {BL_EPI_ADD, t[1]}; return true; }
        if (t[1] == chain && t[0] != chain) { step = {BL_EPI_ADD, t[0]}; return true; }
        return false;
    case BLI_OP_RELU: if (t[0] == chain) { step = {BL_EPI_RELU}; return true; } return false;
    case BLI_OP_GELU: if (t[0] == chain) { step = {BL_EPI_GELU}; return true; } return false;
    case BLI_OP_GELU_ERF: if (t[0] == chain) { step = {BL_EPI_GELU_ERF}; return true; } return false;
    case BLI_OP_SCALE: if (t[0] == chain) { step = {BL_EPI_SCALE, BLI_NONE, o.f}; return true; } return false;
    case BLI_OP_CHANNEL_SCALE:
        if (t[0] == chain && t[1] != chain) { step = {BL_EPI_CHANNEL_SCALE, t[1], 0.0f, o.d[1]}; return true; }
        return false;
    default: return false;
    }
}

// ---- KernelSpec (kernel.rs:1937-2264) ----

struct Spec {
    MainOp main;
    std::vector<Epi> epilogue;
    uint32_t output = BLI_NONE;
    uint32_t op_begin = 0, op_end = 0;
    uint32_t part_index = 0, part_count = 1, part_start = 0, part_end = 0;
    uint32_t prologue = 0;  // BL_PRO_* applied to the main input as it is loaded (kernel.rs:1639-1659)

    static Spec whole_of(const MainOp &m, const std::vector<Epi> &e, uint32_t out, uint32_t b, uint32_t en) {
        Spec s;
        s.main = m;
        s.epilogue = e;
        s.output = out;
        s.op_begin = b;
        s.op_end = en;
        s.part_start = 0;
        s.part_end = m.split_extent();
        return s;
    }
    Spec whole() const {
        Spec w = whole_of(main, epilogue, output, op_begin, op_end);
        w.prologue = prologue;
        return w;
    }
    bool is_whole() const { return part_count == 1; }
    uint32_t max_parts() const {  // kernel.rs:1966-1969
        uint32_t g = main.split_grain();
        return (uint32_t)(((uint64_t)main.split_extent() + g - 1) / g);
    }
    // bindings(): main reads, epilogue operands, output; each once (kernel.rs:2096-2113).
    std::vector<uint32_t> bindings() const {
        std::vector<uint32_t> out;
        auto add = [&](uint32_t id) {
            if (std::find(out.begin(), out.end(), id) == out.end()) out.push_back(id);
        };
        for (uint32_t r : main.reads()) add(r);
        for (const Epi &e : epilogue)
            if (e.tensor != BLI_NONE) add(e.tensor);
        out.push_back(output);
        return out;
    }
    std::string name() const {  // KernelSpec::name (kernel.rs:2119-2131): prologue-main+epilogue
        std::string n = prologue == BL_PRO_RELU ? "relu-" : "";
        n += main.name();
        for (const Epi &e : epilogue) {
            n += "+";
            n += epi_name(e.kind);
        }
        return n;
    }
    // Spec::split (kernel.rs:2006-2030).
    std::vector<Spec> split(uint32_t count) const {
        Spec w = whole();
        const uint32_t maxp = std::max<uint32_t>(1, max_parts());
        count = std::min(std::max<uint32_t>(count, 1), maxp);
        const uint32_t extent = main.split_extent(), grain = main.split_grain();
        const uint64_t blocks = max_parts();
        auto edge = [&](uint32_t i) {
            uint64_t block = blocks * i / count;
            uint64_t unit = block * grain;
            return (uint32_t)std::min<uint64_t>(unit, extent);
        };
        std::vector<Spec> parts;
        for (uint32_t i = 0; i < count; i++) {
            Spec p = w;
            p.part_index = i;
            p.part_count = count;
            p.part_start = edge(i);
            p.part_end = edge(i + 1);
            parts.push_back(p);
        }
        return parts;
    }
};

// rows_of (kernel.rs:2267-2273): a 1-D workgroup count as rows of the baseline's width.
void rows_of(uint64_t groups, uint32_t max_dim, uint32_t out[3]) {
    uint64_t g = std::max<uint64_t>(groups, 1);
    uint64_t width = std::min<uint64_t>(max_dim, g);
    out[0] = (uint32_t)width;
    out[1] = (uint32_t)((g + width - 1) / width);
    out[2] = 1;
}

// KernelSpec::requirements + check (kernel.rs:2118-2244) for the baseline variant.
int check_spec(const Spec &s, const bli_profile &p) {
    const uint32_t units = s.part_end - s.part_start;
    uint32_t wg[3] = {1, 1, 1}, groups[3] = {1, 1, 1}, storage = 0;
    uint32_t cols, layers;
    if (s.main.tile_columns_and_layers(cols, layers)) {
        const uint32_t tc = s.main.tile_columns();
        wg[0] = tc / 4;
        wg[1] = TILE_ROWS / 4;
        groups[0] = (cols + tc - 1) / tc;
        groups[1] = (units + TILE_ROWS - 1) / TILE_ROWS;
        groups[2] = layers;
        storage = 16 * ((TILE_ROWS + 4) + (tc + 4)) * 4;
    } else if (s.main.kind == BL_MAIN_LAYER_NORM) {
        wg[0] = LAYER_NORM_LANES;
        rows_of(units, p.max_compute_workgroups_per_dimension, groups);
        storage = LAYER_NORM_LANES * 4;
    } else if (s.main.kind == BL_MAIN_SOFTMAX) {
        wg[0] = SOFTMAX_LANES;
        rows_of(units, p.max_compute_workgroups_per_dimension, groups);
        storage = SOFTMAX_LANES * 4;
    } else if (s.main.kind == BL_MAIN_FLASH_ATTENTION) {
        // The HIP kernel: 256 invocations per 64 query rows and head.
        wg[0] = 256;
        groups[0] = (units + 63) / 64;
        groups[1] = s.main.d[1];
    } else {
        wg[0] = ELEMENT_GROUP;
        uint64_t elements = (uint64_t)units * s.main.elements_per_unit();
        rows_of((elements + ELEMENT_GROUP - 1) / ELEMENT_GROUP, p.max_compute_workgroups_per_dimension, groups);
    }
    const uint32_t buffers = (uint32_t)s.bindings().size();
    auto over = [&](const char *limit, uint64_t need, uint64_t have) {
        return err(BLI_ERR_EXCEEDS_LIMIT, "the kernel %s needs %llu of %s, the device provides %llu", s.name().c_str(),
                   (unsigned long long)need, limit, (unsigned long long)have);
    };
    if (storage > p.max_compute_workgroup_storage_size) return over("WorkgroupStorageSize", storage, p.max_compute_workgroup_storage_size);
    if ((uint64_t)wg[0] * wg[1] * wg[2] > p.max_compute_invocations_per_workgroup)
        return over("InvocationsPerWorkgroup", (uint64_t)wg[0] * wg[1] * wg[2], p.max_compute_invocations_per_workgroup);
    for (uint32_t c : groups)
        if (c > p.max_compute_workgroups_per_dimension) return over("WorkgroupsPerDimension", c, p.max_compute_workgroups_per_dimension);
    if (buffers > p.max_storage_buffers_per_shader_stage)
        return over("StorageBuffersPerShaderStage", buffers, p.max_storage_buffers_per_shader_stage);
    return 0;
}

const bli_profile BASELINE = {128ull << 20, 256ull << 20, 256, 16384, 256, 65535, 8};

}  // namespace

// ---- the C API's objects ----

struct bli_graph {
    std::map<uint32_t, TensorInfo> tensors;
    std::vector<std::pair<bli_op, uint32_t>> ops;  // (kind, output)
    std::set<uint32_t> written;
};

struct bli_program {
    std::vector<Spec> kernels;
    std::vector<bli_tensor_desc> tensors;
    std::map<uint32_t, TensorInfo> infos;
};

struct bli_plan {
    std::vector<uint64_t> arenas;
    std::map<uint32_t, bli_placement> placements;
    uint64_t peak = 0;
    uint64_t alignment = 0;
};

namespace {

// Program::derive (kernel.rs:2294-2333): lifetimes from the kernels that bind each tensor.
bli_program *derive(std::vector<Spec> kernels, const std::map<uint32_t, TensorInfo> &infos, uint32_t dtype) {
    auto *p = new bli_program();
    const uint32_t last = kernels.empty() ? 0 : (uint32_t)kernels.size() - 1;
    std::map<uint32_t, std::pair<uint32_t, uint32_t>> uses;
    for (uint32_t k = 0; k < kernels.size(); k++)
        for (uint32_t id : kernels[k].bindings()) {
            auto it = uses.find(id);
            if (it == uses.end()) uses[id] = {k, k};
            else {
                it->second.first = std::min(it->second.first, k);
                it->second.second = std::max(it->second.second, k);
            }
        }
    for (const auto &[id, info] : infos) {
        bool have = false;
        uint32_t first = 0, end = 0;
        if (role_whole_program(info.role)) {
            have = true;
            first = 0;
            end = last;
        } else if (auto it = uses.find(id); it != uses.end()) {
            have = true;
            first = it->second.first;
            end = it->second.second;
        }
        if (have) {
            p->tensors.push_back(bli_tensor_desc{id, dtype, info.elements, first, end});
            p->infos[id] = info;
        }
    }
    p->kernels = std::move(kernels);
    return p;
}

uint32_t program_dtype(const bli_program *p) { return p->tensors.empty() ? BL_F32 : p->tensors[0].dtype; }

}  // namespace

extern "C" const char *bli_last_error(void) { return g_error.c_str(); }

extern "C" void bli_profile_webgpu_baseline(bli_profile *out) { *out = BASELINE; }

// The HIP backend's limits: arenas as large as the device (288 GB of HBM3E on
// an MI355X; kernels address with 64-bit offsets), 256-byte placement
// alignment, 160 KB of LDS per CU (64 KB per workgroup), 1024 invocations per
// workgroup, and no binding-count limit below the spec's 8 bindings.
extern "C" void bli_profile_mi355x(bli_profile *out) {
    *out = bli_profile{288ull << 30, 288ull << 30, 256, 65536, 1024, 0x7fffffffu, 8};
}

extern "C" int bli_graph_new(bli_graph **out) {
    *out = new bli_graph();
    return 0;
}
extern "C" void bli_graph_free(bli_graph *g) { delete g; }
extern "C" uint32_t bli_graph_ops(const bli_graph *g) { return (uint32_t)g->ops.size(); }
extern "C" uint64_t bli_op_output_elements(const bli_op *op) { return op_output(*op); }

// Graph::tensor (kernel.rs:1151-1169).
extern "C" int bli_graph_tensor(bli_graph *g, uint32_t id, uint32_t role, uint64_t elements) {
    if (g->tensors.count(id)) return err(BLI_ERR_DUPLICATE_TENSOR, "tensor %u is declared more than once", id);
    if (elements == 0) return err(BLI_ERR_EMPTY_TENSOR, "tensor %u has no elements", id);
    if (elements > MAX_ELEMENTS) return err(BLI_ERR_TENSOR_TOO_LARGE, "tensor %u has more than %llu elements", id, (unsigned long long)MAX_ELEMENTS);
    if (role > BLI_OUTPUT) return err(BLI_ERR_UNKNOWN_OP, "unknown role %u", role);
    g->tensors[id] = TensorInfo{role, elements};
    return 0;
}

// Graph::push (kernel.rs:1181-1228).
extern "C" int bli_graph_push(bli_graph *g, const bli_op *op_in, uint32_t output) {
    const bli_op &op = *op_in;
    const size_t index = g->ops.size();
    if (index + 1 > UINT32_MAX) return err(BLI_ERR_TOO_MANY_OPS, "too many operations");
    if (op_reads(op).empty()) return err(BLI_ERR_UNKNOWN_OP, "operation %zu: unknown kind %u", index, op.kind);
    if (op.kind == BLI_OP_SCALE && !std::isfinite(op.f))
        return err(BLI_ERR_NON_FINITE_SCALE, "operation %zu scales by a non-finite factor", index);
    if (op.kind == BLI_OP_LAYER_NORM && !(std::isfinite(op.f) && op.f > 0.0f))
        return err(BLI_ERR_INVALID_EPSILON, "operation %zu is a layer norm whose epsilon is not finite and positive", index);
    if (op_has_zero_dim(op)) return err(BLI_ERR_ZERO_DIMENSION, "operation %zu has a zero dimension", index);
    const uint64_t out_elements = op_output(op);
    const auto reads = op_reads(op);
    bool too_large = out_elements > MAX_ELEMENTS;
    for (auto &r : reads) too_large |= r.second > MAX_ELEMENTS;
    if (too_large) return err(BLI_ERR_OP_TOO_LARGE, "operation %zu has a tensor of more than %llu elements", index, (unsigned long long)MAX_ELEMENTS);
    auto info = [&](uint32_t id, uint64_t expected, TensorInfo &ti) -> int {
        auto it = g->tensors.find(id);
        if (it == g->tensors.end()) return err(BLI_ERR_UNKNOWN_TENSOR, "tensor %u is not declared", id);
        if (it->second.elements != expected)
            return err(BLI_ERR_ELEMENT_COUNT, "tensor %u has %llu elements, but operation %zu needs %llu", id,
                       (unsigned long long)it->second.elements, index, (unsigned long long)expected);
        ti = it->second;
        return 0;
    };
    for (auto &[tensor, expected] : reads) {
        TensorInfo ti;
        if (int r = info(tensor, expected, ti)) return r;
        if (role_written_by_op(ti.role) && !g->written.count(tensor))
            return err(BLI_ERR_READ_BEFORE_WRITTEN, "operation %zu reads tensor %u before any operation writes it", index, tensor);
    }
    TensorInfo ti;
    if (int r = info(output, out_elements, ti)) return r;
    if (!role_written_by_op(ti.role))
        return err(BLI_ERR_NOT_WRITABLE, "operation %zu writes tensor %u, an input or weight", index, output);
    if (!g->written.insert(output).second)
        return err(BLI_ERR_WRITTEN_TWICE, "operation %zu writes tensor %u, which an earlier operation wrote", index, output);
    g->ops.push_back({op, output});
    return 0;
}

// Graph::lower + fuse (kernel.rs:1285-1375), rule 2: an element-wise operation
// folds into the previous heavy kernel when it reads that kernel's output and
// nothing else does, and the bindings stay within the baseline's limit.
extern "C" int bli_graph_lower(const bli_graph *g, uint32_t fusion, bli_program **out) {
    *out = nullptr;
    if (g->ops.empty()) return err(BLI_ERR_EMPTY_GRAPH, "the graph has no operations");
    for (const auto &[id, t] : g->tensors)
        if (role_written_by_op(t.role) && !g->written.count(id)) return err(BLI_ERR_NEVER_WRITTEN, "tensor %u is never written", id);
    std::map<uint32_t, size_t> consumers;
    for (const auto &[op, o] : g->ops)
        for (auto &r : op_reads(op)) consumers[r.first]++;
    std::vector<Spec> kernels;
    // relu_prologue (kernel.rs:1381-1402): a ReLU whose output is an
    // activation read once, by the 3x3 convolution right after it as its
    // image, becomes that convolution's prologue; the convolution binds the
    // ReLU's input instead.
    auto relu_prologue = [&](uint32_t index) {
        const bli_op &op = g->ops[index].first;
        if (op.kind != BLI_OP_RELU || index + 1 >= g->ops.size()) return false;
        const uint32_t relu = g->ops[index].second;
        const bli_op &next = g->ops[index + 1].first;
        auto role = g->tensors.find(relu);
        return next.kind == BLI_OP_CONV3X3 && next.t[0] == relu && role != g->tensors.end() &&
               role->second.role == BLI_ACTIVATION && consumers[relu] == 1;
    };
    bool deferred = false;
    uint32_t deferred_at = 0, deferred_input = BLI_NONE;
    for (uint32_t index = 0; index < g->ops.size(); index++) {
        const bli_op &op = g->ops[index].first;
        const uint32_t output = g->ops[index].second;
        if (fusion == BLI_FUSION_ON && !kernels.empty()) {
            Spec &last = kernels.back();
            const uint32_t chain = last.output;
            auto role = g->tensors.find(chain);
            Epi step{};
            if (last.main.kind != BL_MAIN_MAP && role != g->tensors.end() && role->second.role == BLI_ACTIVATION &&
                consumers[chain] == 1 && as_epilogue(op, chain, step)) {
                Spec fused = last;
                fused.epilogue.push_back(step);
                fused.output = output;
                if (fused.bindings().size() <= BASELINE.max_storage_buffers_per_shader_stage) {
                    fused.op_end = index + 1;
                    fused.part_end = fused.main.split_extent();
                    last = fused;
                    continue;
                }
            }
        }
        if (fusion == BLI_FUSION_ON && relu_prologue(index)) {
            deferred = true;
            deferred_at = index;
            deferred_input = op.t[0];
            continue;
        }
        MainOp m;
        std::vector<Epi> e;
        standalone(op, m, e);
        uint32_t start = index, prologue = 0;
        if (deferred) {
            m.t[0] = deferred_input;
            prologue = BL_PRO_RELU;
            start = deferred_at;
            deferred = false;
        }
        kernels.push_back(Spec::whole_of(m, e, output, start, index + 1));
        kernels.back().prologue = prologue;
    }
    for (const Spec &s : kernels)
        if (int r = check_spec(s, BASELINE)) return r;
    *out = derive(std::move(kernels), g->tensors, BL_F32);
    return 0;
}

extern "C" void bli_program_free(bli_program *p) { delete p; }

// Program::split (kernel.rs:2384-2408), rule 6.
extern "C" int bli_program_split(const bli_program *p, const uint32_t *parts, uint32_t n, bli_program **out) {
    *out = nullptr;
    if (n != p->kernels.size()) return err(BLI_ERR_PART_COUNTS, "%u entries given for a program of %zu kernels", n, p->kernels.size());
    uint64_t total = 0;
    for (uint32_t i = 0; i < n; i++) {
        if (!p->kernels[i].is_whole()) return err(BLI_ERR_ALREADY_SPLIT, "kernel %u is already a part of a split kernel", i);
        total += std::min(std::max<uint32_t>(parts[i], 1), std::max<uint32_t>(p->kernels[i].max_parts(), 1));
    }
    if (total > UINT32_MAX) return err(BLI_ERR_TOO_MANY_OPS, "too many operations");
    std::vector<Spec> kernels;
    for (uint32_t i = 0; i < n; i++)
        for (Spec &s : p->kernels[i].split(parts[i])) kernels.push_back(s);
    *out = derive(std::move(kernels), p->infos, program_dtype(p));
    return 0;
}

// Program::parts_within (kernel.rs:2350-2366): ceil(duration / bound) in 1..=max_parts.
extern "C" int bli_program_parts_within(const bli_program *p, const uint64_t *durations, uint32_t n, uint64_t bound,
                                        uint32_t *parts_out) {
    if (n != p->kernels.size()) return err(BLI_ERR_PART_COUNTS, "%u entries given for a program of %zu kernels", n, p->kernels.size());
    if (bound == 0) return err(BLI_ERR_ZERO_BOUND, "a dispatch bound of zero cannot be met");
    for (uint32_t i = 0; i < n; i++) {
        const uint64_t d = durations[i];
        uint64_t wanted = std::max<uint64_t>(d / bound + (d % bound != 0), 1);
        parts_out[i] = (uint32_t)std::min<uint64_t>(wanted, std::max<uint32_t>(p->kernels[i].max_parts(), 1));
    }
    return 0;
}

// The backend's rewrite: attention_scores(+scale) -> softmax -> attention_values
// over one qkv tensor, whole, with no other reader of the scores or the
// probabilities, becomes one flash_attention kernel.
extern "C" int bli_program_fuse_attention(const bli_program *p, bli_program **out) {
    std::map<uint32_t, int> readers;
    for (const Spec &s : p->kernels)
        for (uint32_t id : s.bindings())
            if (id != s.output) readers[id]++;
    std::vector<Spec> kernels;
    for (size_t i = 0; i < p->kernels.size(); i++) {
        const Spec &a = p->kernels[i];
        if (i + 2 < p->kernels.size() && a.main.kind == BL_MAIN_ATTENTION_SCORES && a.is_whole()) {
            const Spec &b = p->kernels[i + 1], &c = p->kernels[i + 2];
            bool scale_only = a.epilogue.empty() || (a.epilogue.size() == 1 && a.epilogue[0].kind == BL_EPI_SCALE);
            auto role_of = [&](uint32_t id) { auto it = p->infos.find(id); return it == p->infos.end() ? BLI_NONE : it->second.role; };
            if (scale_only && b.main.kind == BL_MAIN_SOFTMAX && b.is_whole() && b.epilogue.empty() &&
                b.main.t[0] == a.output && c.main.kind == BL_MAIN_ATTENTION_VALUES && c.is_whole() &&
                c.epilogue.empty() && c.main.t[0] == b.output && c.main.t[1] == a.main.t[0] &&
                a.main.d[2] == 64 && readers[a.output] == 1 && readers[b.output] == 1 &&
                role_of(a.output) == BLI_ACTIVATION && role_of(b.output) == BLI_ACTIVATION) {
                MainOp m;
                m.kind = BL_MAIN_FLASH_ATTENTION;
                m.t[0] = a.main.t[0];
                m.d[0] = a.main.d[0];
                m.d[1] = a.main.d[1];
                m.d[2] = a.main.d[2];
                m.scale = a.epilogue.empty() ? 1.0f : a.epilogue[0].factor;
                kernels.push_back(Spec::whole_of(m, {}, c.output, a.op_begin, c.op_end));
                i += 2;
                continue;
            }
        }
        kernels.push_back(a);
    }
    *out = derive(std::move(kernels), p->infos, program_dtype(p));
    return 0;
}

extern "C" int bli_program_set_dtype(bli_program *p, uint32_t dtype) {
    if (dtype != BL_F32 && dtype != BL_F16) return err(BLI_ERR_UNKNOWN_OP, "unknown dtype %u", dtype);
    for (auto &t : p->tensors) t.dtype = dtype;
    return 0;
}

extern "C" uint32_t bli_program_len(const bli_program *p) { return (uint32_t)p->kernels.size(); }

extern "C" int bli_program_kernel(const bli_program *p, uint32_t k, bli_kernel_info *out) {
    if (k >= p->kernels.size()) return err(BLI_ERR_UNKNOWN_OP, "there is no kernel %u", k);
    const Spec &s = p->kernels[k];
    memset(out, 0, sizeof *out);
    out->main = s.main.kind;
    memcpy(out->dims, s.main.d, sizeof out->dims);
    out->epsilon = s.main.eps;
    out->scale = s.main.scale;
    out->part = bl_part{s.part_index, s.part_count, s.part_start, s.part_end};
    out->max_parts = s.max_parts();
    out->tile_rows = s.main.split_grain() > 1 ? s.main.split_grain() : 0;
    out->output_start = (uint64_t)s.part_start * s.main.elements_per_unit();
    out->output_end = (uint64_t)s.part_end * s.main.elements_per_unit();
    const std::vector<uint32_t> b = s.bindings();
    auto index_of = [&](uint32_t id) { return (uint32_t)(std::find(b.begin(), b.end(), id) - b.begin()); };
    const auto reads = s.main.reads();
    out->n_reads = (uint32_t)reads.size();
    for (size_t i = 0; i < reads.size(); i++) out->reads[i] = index_of(reads[i]);
    out->n_epilogue = (uint32_t)s.epilogue.size();
    for (size_t i = 0; i < s.epilogue.size() && i < BL_MAX_EPILOGUE; i++) {
        const Epi &e = s.epilogue[i];
        out->epilogue[i] = bl_epilogue{e.kind, e.factor, e.channels, e.tensor == BLI_NONE ? 0u : index_of(e.tensor)};
    }
    out->n_bindings = (uint32_t)b.size();
    for (size_t i = 0; i < b.size() && i < BL_MAX_BINDINGS; i++) out->bindings[i] = b[i];
    out->first_op = s.op_begin;
    out->end_op = s.op_end;
    out->prologue = s.prologue;
    return 0;
}

extern "C" int bli_program_kernel_name(const bli_program *p, uint32_t k, char *buf, uint32_t cap) {
    if (k >= p->kernels.size()) return err(BLI_ERR_UNKNOWN_OP, "there is no kernel %u", k);
    snprintf(buf, cap, "%s", p->kernels[k].name().c_str());
    return 0;
}

extern "C" uint32_t bli_program_tensors(const bli_program *p, bli_tensor_desc *out, uint32_t cap) {
    for (uint32_t i = 0; i < p->tensors.size() && i < cap; i++) out[i] = p->tensors[i];
    return (uint32_t)p->tensors.size();
}

extern "C" int bli_program_role(const bli_program *p, uint32_t id) {
    auto it = p->infos.find(id);
    return it == p->infos.end() ? -1 : (int)it->second.role;
}

// Program::stand_in (kernel.rs:2427-2451).
extern "C" int bli_program_stand_in(const bli_program *p, uint32_t of, uint32_t id, bli_tensor_desc *out) {
    if (p->infos.count(id)) return err(BLI_ERR_DUPLICATE_TENSOR, "tensor %u is declared more than once", id);
    auto it = p->infos.find(of);
    if (it != p->infos.end() && (it->second.role == BLI_INPUT || it->second.role == BLI_OUTPUT))
        for (const auto &t : p->tensors)
            if (t.id == of) {
                *out = t;
                out->id = id;
                return 0;
            }
    return err(BLI_ERR_NOT_INPUT_OR_OUTPUT, "tensor %u is not an input or output of the program", of);
}

extern "C" int bli_program_spec(const bli_program *p, uint32_t k, const bli_plan *plan, bl_spec *out) {
    bli_kernel_info info;
    if (int r = bli_program_kernel(p, k, &info)) return r;
    memset(out, 0, sizeof *out);
    out->main = info.main;
    memcpy(out->dims, info.dims, sizeof out->dims);
    out->epsilon = info.epsilon;
    out->scale = info.scale;
    out->part = info.part;
    out->n_reads = info.n_reads;
    memcpy(out->reads, info.reads, sizeof out->reads);
    out->n_epilogue = info.n_epilogue;
    memcpy(out->epilogue, info.epilogue, sizeof out->epilogue);
    out->n_bindings = info.n_bindings;
    out->prologue = info.prologue;
    const uint32_t dtype = program_dtype(p);
    for (uint32_t b = 0; b < info.n_bindings; b++) {
        auto it = plan->placements.find(info.bindings[b]);
        if (it == plan->placements.end()) return err(BLI_ERR_NO_PLACEMENT, "tensor %u has no placement in the memory plan", info.bindings[b]);
        out->bindings[b] = bl_binding{info.bindings[b], it->second.arena, it->second.offset, it->second.size, dtype, 0};
    }
    return 0;
}

// ---- MemoryPlan (memory.rs:266-499) ----

namespace {
uint64_t max_arena(const bli_profile &p) { return std::min(p.max_storage_buffer_binding_size, p.max_buffer_size); }
bool round_up(uint64_t v, uint64_t m, uint64_t &out) {
    uint64_t r = v % m;
    if (r == 0) { out = v; return true; }
    if (v > UINT64_MAX - (m - r)) return false;
    out = v + (m - r);
    return true;
}
struct Sized {
    bli_tensor_desc d;
    uint64_t size;
};
bool overlaps(const bli_tensor_desc &a, const bli_tensor_desc &b) { return a.first_use <= b.last_use && b.first_use <= a.last_use; }
}  // namespace

extern "C" int bli_plan_new(const bli_tensor_desc *tensors, uint32_t n, const bli_profile *profile, bli_plan **out) {
    *out = nullptr;
    const uint64_t alignment = profile->min_storage_buffer_offset_alignment, cap = max_arena(*profile);
    if (alignment == 0 || cap == 0) return err(BLI_ERR_PLAN_INVALID_PROFILE, "the device profile has a zero offset alignment or a zero arena size");
    std::set<uint32_t> seen;
    std::vector<Sized> sized;
    for (uint32_t i = 0; i < n; i++) {
        const bli_tensor_desc &d = tensors[i];
        if (!seen.insert(d.id).second) return err(BLI_ERR_PLAN_DUPLICATE_TENSOR, "tensor %u is described more than once", d.id);
        if (d.first_use > d.last_use)
            return err(BLI_ERR_PLAN_INVALID_LIFETIME, "tensor %u is first used at operation %u, after its last use at %u", d.id, d.first_use, d.last_use);
        if (d.elements == 0) return err(BLI_ERR_PLAN_EMPTY_TENSOR, "tensor %u has no elements", d.id);
        const uint64_t esz = d.dtype == BL_F16 ? 2 : 4;
        uint64_t size;
        if (d.elements > UINT64_MAX / esz || !round_up(d.elements * esz, 4, size))
            return err(BLI_ERR_PLAN_SIZE_OVERFLOW, "the size of tensor %u overflows", d.id);
        if (size > cap)
            return err(BLI_ERR_PLAN_TENSOR_TOO_LARGE, "tensor %u needs %llu bytes but an arena holds at most %llu", d.id,
                       (unsigned long long)size, (unsigned long long)cap);
        sized.push_back({d, size});
    }
    auto *plan = new bli_plan();
    plan->alignment = alignment;
    // peak_live (memory.rs:486-503)
    std::map<uint64_t, std::pair<uint64_t, uint64_t>> deltas;
    for (const Sized &s : sized) {
        deltas[s.d.first_use].first += s.size;
        deltas[(uint64_t)s.d.last_use + 1].second += s.size;
    }
    uint64_t live = 0;
    for (auto &[at, ar] : deltas) {
        live = live + ar.first - std::min(live + ar.first, ar.second);
        plan->peak = std::max(plan->peak, live);
    }
    // Greedy by size, descending, ties by id; lowest aligned fit in the first arena that has one.
    std::sort(sized.begin(), sized.end(), [](const Sized &a, const Sized &b) {
        return a.size != b.size ? a.size > b.size : a.d.id < b.d.id;
    });
    std::vector<std::vector<std::pair<bli_tensor_desc, std::pair<uint64_t, uint64_t>>>> arenas;
    for (const Sized &item : sized) {
        int found = -1;
        uint64_t offset = 0;
        for (size_t a = 0; a < arenas.size() && found < 0; a++) {
            std::vector<std::pair<uint64_t, uint64_t>> busy;
            for (auto &[d, r] : arenas[a])
                if (overlaps(d, item.d)) busy.push_back({r.first, r.first + r.second});
            std::sort(busy.begin(), busy.end());
            uint64_t candidate = 0;
            bool ok = true;
            for (auto [start, end] : busy) {
                uint64_t aligned;
                if (!round_up(candidate, alignment, aligned)) { ok = false; break; }
                if (aligned + item.size <= start) break;
                candidate = std::max(candidate, end);
            }
            uint64_t off;
            if (ok && round_up(candidate, alignment, off) && off + item.size <= cap) {
                found = (int)a;
                offset = off;
            }
        }
        if (found < 0) {
            arenas.emplace_back();
            found = (int)arenas.size() - 1;
            offset = 0;
        }
        arenas[found].push_back({item.d, {offset, item.size}});
        plan->placements[item.d.id] = bli_placement{(uint32_t)found, 0, offset, item.size};
    }
    for (auto &a : arenas) {
        uint64_t size = 0;
        for (auto &[d, r] : a) size = std::max(size, r.first + r.second);
        plan->arenas.push_back(size);
    }
    *out = plan;
    return 0;
}

extern "C" void bli_plan_free(bli_plan *plan) { delete plan; }
extern "C" uint32_t bli_plan_arenas(const bli_plan *plan, uint64_t *sizes, uint32_t cap) {
    for (uint32_t i = 0; i < plan->arenas.size() && i < cap; i++) sizes[i] = plan->arenas[i];
    return (uint32_t)plan->arenas.size();
}
extern "C" int bli_plan_placement(const bli_plan *plan, uint32_t id, bli_placement *out) {
    auto it = plan->placements.find(id);
    if (it == plan->placements.end()) return err(BLI_ERR_NO_PLACEMENT, "tensor %u has no placement in the memory plan", id);
    *out = it->second;
    return 0;
}
extern "C" uint64_t bli_plan_peak_live_bytes(const bli_plan *plan) { return plan->peak; }
extern "C" uint64_t bli_plan_total_bytes(const bli_plan *plan) {
    uint64_t s = 0;
    for (uint64_t a : plan->arenas) s += a;
    return s;
}
// MemoryPlan::valid_on (memory.rs:421-428).
extern "C" int bli_plan_valid_on(const bli_plan *plan, const bli_profile *profile) {
    const uint64_t a = profile->min_storage_buffer_offset_alignment;
    if (a == 0 || plan->alignment % a) return 0;
    for (uint64_t s : plan->arenas)
        if (s > max_arena(*profile)) return 0;
    return 1;
}

// ---- model (crates/beatlm/src/model/depth_anything_v2.rs) ----

// layer_of (depth_anything_v2.rs:264-424): the pre-norm DINOv2 layer,
//   x1  = x  + ls1 * proj(attention(norm1(x)))
//   out = x1 + ls2 * fc2(gelu_erf(fc1(norm2(x1))))
// weights declared first, then one tensor per operation, ids handed out in order.
extern "C" int bli_vit_block(bli_graph *g, const bli_vit_dims *d, uint32_t x, uint32_t first_id, uint32_t out_role,
                             bli_block_ids *ids) {
    const uint32_t T = d->tokens, D = d->width, H = d->heads, M = d->mlp;
    if (!H || D % H) return err(BLI_ERR_ZERO_DIMENSION, "width %u is not a whole number of %u heads", D, H);
    const uint32_t HD = D / H;
    uint32_t next = first_id;
    auto weight = [&](uint64_t elements, uint32_t &id) {
        id = next++;
        return bli_graph_tensor(g, id, BLI_WEIGHT, elements);
    };
    int r;
    if ((r = weight(D, ids->norm1_g)) || (r = weight(D, ids->norm1_b)) || (r = weight((uint64_t)D * 3 * D, ids->qkv_w)) ||
        (r = weight(3 * D, ids->qkv_b)) || (r = weight((uint64_t)D * D, ids->proj_w)) || (r = weight(D, ids->proj_b)) ||
        (r = weight(D, ids->ls1)) || (r = weight(D, ids->norm2_g)) || (r = weight(D, ids->norm2_b)) ||
        (r = weight((uint64_t)D * M, ids->fc1_w)) || (r = weight(M, ids->fc1_b)) || (r = weight((uint64_t)M * D, ids->fc2_w)) ||
        (r = weight(D, ids->fc2_b)) || (r = weight(D, ids->ls2)))
        return r;
    auto op = [&](bli_op o, uint32_t role, uint32_t &out) {
        out = next++;
        int rc = bli_graph_tensor(g, out, role, op_output(o));
        return rc ? rc : bli_graph_push(g, &o, out);
    };
    const uint32_t N = BLI_NONE;
    uint32_t n1, qkv, scores, scaled, probs, values, projected, scaled1, x1, n2, hidden, act, fc2o, scaled2, y;
    if ((r = op(bli_op{BLI_OP_LAYER_NORM, {x, ids->norm1_g, ids->norm1_b, N}, {T, D}, d->epsilon}, BLI_ACTIVATION, n1)) ||
        (r = op(bli_op{BLI_OP_MATMUL, {n1, ids->qkv_w, ids->qkv_b, N}, {T, D, 3 * D}}, BLI_ACTIVATION, qkv)) ||
        (r = op(bli_op{BLI_OP_ATTENTION_SCORES, {qkv, N, N, N}, {T, H, HD}}, BLI_ACTIVATION, scores)) ||
        (r = op(bli_op{BLI_OP_SCALE, {scores, N, N, N}, {T * H * T}, 1.0f / std::sqrt((float)HD)}, BLI_ACTIVATION, scaled)) ||
        (r = op(bli_op{BLI_OP_SOFTMAX, {scaled, N, N, N}, {T * H, T}}, BLI_ACTIVATION, probs)) ||
        (r = op(bli_op{BLI_OP_ATTENTION_VALUES, {probs, qkv, N, N}, {T, H, HD}}, BLI_ACTIVATION, values)) ||
        (r = op(bli_op{BLI_OP_MATMUL, {values, ids->proj_w, ids->proj_b, N}, {T, D, D}}, BLI_ACTIVATION, projected)) ||
        (r = op(bli_op{BLI_OP_CHANNEL_SCALE, {projected, ids->ls1, N, N}, {T, D}}, BLI_ACTIVATION, scaled1)) ||
        (r = op(bli_op{BLI_OP_ADD, {scaled1, x, N, N}, {T * D}}, BLI_ACTIVATION, x1)) ||
        (r = op(bli_op{BLI_OP_LAYER_NORM, {x1, ids->norm2_g, ids->norm2_b, N}, {T, D}, d->epsilon}, BLI_ACTIVATION, n2)) ||
        (r = op(bli_op{BLI_OP_MATMUL, {n2, ids->fc1_w, ids->fc1_b, N}, {T, D, M}}, BLI_ACTIVATION, hidden)) ||
        (r = op(bli_op{BLI_OP_GELU_ERF, {hidden, N, N, N}, {T * M}}, BLI_ACTIVATION, act)) ||
        (r = op(bli_op{BLI_OP_MATMUL, {act, ids->fc2_w, ids->fc2_b, N}, {T, M, D}}, BLI_ACTIVATION, fc2o)) ||
        (r = op(bli_op{BLI_OP_CHANNEL_SCALE, {fc2o, ids->ls2, N, N}, {T, D}}, BLI_ACTIVATION, scaled2)) ||
        (r = op(bli_op{BLI_OP_ADD, {scaled2, x1, N, N}, {T * D}}, out_role, y)))
        return r;
    ids->output = y;
    ids->next_id = next;
    return 0;
}

// encoder() up to the first block (depth_anything_v2.rs:446-498): patch
// embedding, class token, position embedding.
extern "C" int bli_vit_embeddings(bli_graph *g, uint32_t grid, uint32_t patch, uint32_t channels, uint32_t width,
                                  uint32_t first_id, bli_embed_ids *ids) {
    uint32_t next = first_id;
    const uint32_t T = grid * grid + 1;
    int r;
    ids->image = next++;
    if ((r = bli_graph_tensor(g, ids->image, BLI_INPUT, product({grid, patch, grid, patch, channels})))) return r;
    ids->patch_w = next++;
    if ((r = bli_graph_tensor(g, ids->patch_w, BLI_WEIGHT, product({patch, patch, channels, width})))) return r;
    ids->patch_b = next++;
    if ((r = bli_graph_tensor(g, ids->patch_b, BLI_WEIGHT, width))) return r;
    ids->cls = next++;
    if ((r = bli_graph_tensor(g, ids->cls, BLI_WEIGHT, width))) return r;
    ids->pos = next++;
    if ((r = bli_graph_tensor(g, ids->pos, BLI_WEIGHT, (uint64_t)T * width))) return r;
    const uint32_t N = BLI_NONE;
    uint32_t patches = next++, tokens = next++, embedded = next++;
    bli_op pe{BLI_OP_PATCH_EMBED, {ids->image, ids->patch_w, ids->patch_b, N}, {grid, grid, patch, channels, width}};
    bli_op pt{BLI_OP_PREPEND_TOKEN, {ids->cls, patches, N, N}, {grid * grid, width}};
    bli_op add{BLI_OP_ADD, {tokens, ids->pos, N, N}, {T * width}};
    if ((r = bli_graph_tensor(g, patches, BLI_ACTIVATION, op_output(pe))) || (r = bli_graph_push(g, &pe, patches)) ||
        (r = bli_graph_tensor(g, tokens, BLI_ACTIVATION, op_output(pt))) || (r = bli_graph_push(g, &pt, tokens)) ||
        (r = bli_graph_tensor(g, embedded, BLI_ACTIVATION, op_output(add))) || (r = bli_graph_push(g, &add, embedded)))
        return r;
    ids->output = embedded;
    ids->next_id = next;
    return 0;
}
