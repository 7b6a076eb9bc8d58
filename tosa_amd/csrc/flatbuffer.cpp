// Bounds-checked reader for `.tosa` FlatBuffers (schema/tosa.fbs:695-768),
// producing the IR the reference builds in Graph::from_flatbuffer
// (src/ir.rs:592-885). Every read is checked against the buffer, so a
// malformed buffer raises Error(ERR_DESERIALIZE) instead of reading out of
// bounds. There is no generated code: tables are walked through their
// vtables directly.
#include <cstring>

#include "ir.h"

namespace tosa {
namespace {

class Reader {
public:
    Reader(const uint8_t* d, size_t n) : d_(d), n_(n) {}

    void need(size_t pos, size_t len) const
    {
        if (pos > n_ || len > n_ - pos)
            throw Error(ERR_DESERIALIZE, "failed to deserialize flatbuffer: read of " + std::to_string(len) +
                                             " bytes at offset " + std::to_string(pos) + " is outside the " +
                                             std::to_string(n_) + "-byte buffer");
    }
    uint8_t u8(size_t p) const { need(p, 1); return d_[p]; }
    uint16_t u16(size_t p) const { need(p, 2); uint16_t v; std::memcpy(&v, d_ + p, 2); return v; }
    uint32_t u32(size_t p) const { need(p, 4); uint32_t v; std::memcpy(&v, d_ + p, 4); return v; }
    int32_t i32(size_t p) const { return static_cast<int32_t>(u32(p)); }

    // Follow the uoffset stored at p.
    size_t deref(size_t p) const
    {
        uint64_t t = static_cast<uint64_t>(p) + u32(p);
        if (t >= n_)
            throw Error(ERR_DESERIALIZE, "failed to deserialize flatbuffer: offset out of range");
        return static_cast<size_t>(t);
    }
    const uint8_t* bytes(size_t p, size_t len) const { need(p, len); return d_ + p; }

private:
    const uint8_t* d_;
    size_t n_;
};

// A table: field(i) is the position of field i, or 0 if absent.
class Table {
public:
    Table(const Reader& r, size_t pos) : r_(r), pos_(pos)
    {
        int64_t vt = static_cast<int64_t>(pos) - r.i32(pos);
        if (vt < 0)
            throw Error(ERR_DESERIALIZE, "failed to deserialize flatbuffer: vtable out of range");
        vt_ = static_cast<size_t>(vt);
        vt_len_ = r.u16(vt_);
        table_len_ = r.u16(vt_ + 2);
        if (vt_len_ < 4 || (vt_len_ & 1))
            throw Error(ERR_DESERIALIZE, "failed to deserialize flatbuffer: malformed vtable");
        r.need(vt_, vt_len_);
        r.need(pos_, table_len_);
    }
    size_t field(int idx) const
    {
        size_t off = 4 + 2 * static_cast<size_t>(idx);
        if (off + 2 > vt_len_)
            return 0;
        uint16_t o = r_.u16(vt_ + off);
        if (o == 0)
            return 0;
        if (o >= table_len_)
            throw Error(ERR_DESERIALIZE, "failed to deserialize flatbuffer: field outside its table");
        return pos_ + o;
    }
    bool has(int idx) const { return field(idx) != 0; }
    uint8_t u8(int idx, uint8_t def = 0) const { size_t p = field(idx); return p ? r_.u8(p) : def; }
    uint32_t u32(int idx, uint32_t def = 0) const { size_t p = field(idx); return p ? r_.u32(p) : def; }
    int32_t i32(int idx, int32_t def = 0) const { size_t p = field(idx); return p ? r_.i32(p) : def; }
    bool boolean(int idx) const { return u8(idx) != 0; }

    std::string str(int idx) const
    {
        size_t p = field(idx);
        if (!p)
            return std::string();
        size_t s = r_.deref(p);
        uint32_t len = r_.u32(s);
        const uint8_t* b = r_.bytes(s + 4, len);
        return std::string(reinterpret_cast<const char*>(b), len);
    }
    // Vector at field idx: (first element position, length); (0,0) if absent.
    std::pair<size_t, uint32_t> vec(int idx, size_t elem) const
    {
        size_t p = field(idx);
        if (!p)
            return {0, 0};
        size_t v = r_.deref(p);
        uint32_t len = r_.u32(v);
        r_.need(v + 4, static_cast<size_t>(len) * elem);
        return {v + 4, len};
    }
    std::vector<int32_t> i32vec(int idx) const
    {
        auto [s, n] = vec(idx, 4);
        std::vector<int32_t> out(n);
        for (uint32_t i = 0; i < n; i++)
            out[i] = r_.i32(s + 4 * i);
        return out;
    }
    std::vector<uint8_t> bytevec(int idx) const
    {
        auto [s, n] = vec(idx, 1);
        if (!n)
            return {};
        const uint8_t* b = r_.bytes(s, n);
        return std::vector<uint8_t>(b, b + n);
    }
    std::vector<std::string> strvec(int idx) const
    {
        auto [s, n] = vec(idx, 4);
        std::vector<std::string> out;
        out.reserve(n);
        for (uint32_t i = 0; i < n; i++) {
            size_t sp = r_.deref(s + 4 * i);
            uint32_t len = r_.u32(sp);
            const uint8_t* b = r_.bytes(sp + 4, len);
            out.emplace_back(reinterpret_cast<const char*>(b), len);
        }
        return out;
    }
    Table sub(size_t elem_pos) const { return Table(r_, r_.deref(elem_pos)); }

private:
    const Reader& r_;
    size_t pos_, vt_ = 0;
    uint16_t vt_len_ = 0, table_len_ = 0;
};

NanMode nan_from(uint32_t v) { return (v == 1 || v == 2) ? static_cast<NanMode>(v) : NAN_UNKNOWN; }
RoundingMode rounding_from(uint32_t v) { return (v >= 1 && v <= 3) ? static_cast<RoundingMode>(v) : ROUND_UNKNOWN; }

// Union type codes of `union Attribute` (schema/tosa.fbs:193-295; NONE = 0).
enum : uint8_t {
    A_ARGMAX = 1, A_AVG_POOL2D = 2, A_CONV2D = 3, A_CONV3D = 4, A_DEPTHWISE = 5, A_FFT2D = 6, A_MAX_POOL2D = 8,
    A_TRANSPOSE_CONV2D = 10, A_CLAMP = 11, A_ARS = 16, A_MAXIMUM = 26, A_MINIMUM = 27, A_REDUCE_ALL = 49,
    A_REDUCE_ANY = 50, A_REDUCE_MAX = 51, A_REDUCE_MIN = 52, A_REDUCE_PRODUCT = 53, A_REDUCE_SUM = 54,
    A_CONCAT = 55, A_REVERSE = 58, A_TRANSPOSE = 61, A_RESIZE = 64, A_RESCALE = 66, A_COND_IF = 70,
    A_WHILE_LOOP = 71, A_DIM = 79, A_ASSERT_EQUAL_SHAPE = 93, A_MAX_POOL2D_ADAPTIVE = 95,
    A_AVG_POOL2D_ADAPTIVE = 96,
};

// src/ir.rs:673-885
OpAttribute parse_attribute(const Table& op)
{
    OpAttribute a;
    uint8_t type = op.u8(1);
    if (!op.has(2))
        return a;
    Table t = op.sub(op.field(2));
    switch (type) {
    case A_COND_IF:
        a.kind = AttrKind::CondIf;
        a.graph_a = t.str(0);
        a.graph_b = t.str(1);
        break;
    case A_WHILE_LOOP:
        a.kind = AttrKind::WhileLoop;
        a.graph_a = t.str(0);
        a.graph_b = t.str(1);
        break;
    case A_CONV2D:
    case A_CONV3D:
    case A_DEPTHWISE:
        a.kind = type == A_CONV2D ? AttrKind::Conv2d : (type == A_CONV3D ? AttrKind::Conv3d : AttrKind::DepthwiseConv2d);
        a.pad = t.i32vec(0);
        a.stride = t.i32vec(1);
        a.dilation = t.i32vec(2);
        a.acc_type = dtype_from_code(t.u32(4));
        break;
    case A_TRANSPOSE_CONV2D:
        a.kind = AttrKind::TransposeConv2d;
        a.out_pad = t.i32vec(0);
        a.stride = t.i32vec(1);
        a.acc_type = dtype_from_code(t.u32(3));
        break;
    case A_AVG_POOL2D:
        a.kind = AttrKind::Pool2d;
        a.kernel = t.i32vec(0);
        a.stride = t.i32vec(1);
        a.pad = t.i32vec(2);
        a.acc_type = dtype_from_code(t.u32(3));
        a.nan_mode = NAN_PROPAGATE;
        break;
    case A_MAX_POOL2D:
        a.kind = AttrKind::Pool2d;
        a.kernel = t.i32vec(0);
        a.stride = t.i32vec(1);
        a.pad = t.i32vec(2);
        a.acc_type = DT_UNKNOWN;
        a.nan_mode = nan_from(t.u32(3));
        break;
    case A_AVG_POOL2D_ADAPTIVE:
        a.kind = AttrKind::Pool2d;
        a.acc_type = dtype_from_code(t.u32(0));
        a.nan_mode = NAN_PROPAGATE;
        break;
    case A_MAX_POOL2D_ADAPTIVE:
        a.kind = AttrKind::Pool2d;
        a.acc_type = DT_UNKNOWN;
        a.nan_mode = nan_from(t.u32(0));
        break;
    case A_ARGMAX:
        a.kind = AttrKind::ArgMax;
        a.axis = t.i32(0);
        a.nan_mode = nan_from(t.u32(1));
        break;
    case A_REDUCE_ALL:
    case A_REDUCE_ANY:
    case A_REDUCE_PRODUCT:
    case A_REDUCE_SUM:
        a.kind = AttrKind::Reduce;
        a.axis = t.i32(0);
        a.nan_mode = NAN_PROPAGATE;
        break;
    case A_REDUCE_MAX:
    case A_REDUCE_MIN:
        a.kind = AttrKind::Reduce;
        a.axis = t.i32(0);
        a.nan_mode = nan_from(t.u32(1));
        break;
    case A_FFT2D:
        a.kind = AttrKind::Fft2d;
        a.flag = t.boolean(0);
        break;
    case A_DIM:
        a.kind = AttrKind::Dim;
        a.axis = t.i32(0);
        break;
    case A_ASSERT_EQUAL_SHAPE:
        a.kind = AttrKind::AssertEqualShape;
        a.flag = t.boolean(0);
        break;
    case A_MAXIMUM:
    case A_MINIMUM:
        a.kind = AttrKind::NanPropagation;
        a.nan_mode = nan_from(t.u32(0));
        break;
    case A_CONCAT:
        a.kind = AttrKind::Concat;
        a.axis = t.i32(0);
        break;
    case A_TRANSPOSE:
        a.kind = AttrKind::Transpose;
        a.perms = t.i32vec(0);
        break;
    case A_CLAMP:
        a.kind = AttrKind::Clamp;
        a.min_val = t.bytevec(0);
        a.max_val = t.bytevec(1);
        a.nan_mode = nan_from(t.u32(2));
        break;
    case A_ARS:
        a.kind = AttrKind::ArithmeticRightShift;
        a.flag = t.boolean(0);
        break;
    case A_RESCALE:
        a.kind = AttrKind::Rescale;
        a.scale32 = t.boolean(0);
        a.rounding_mode = rounding_from(t.u32(1));
        a.per_channel = t.boolean(2);
        a.input_unsigned = t.boolean(3);
        a.output_unsigned = t.boolean(4);
        break;
    case A_REVERSE:
        a.kind = AttrKind::Reverse;
        a.axis = t.i32(0);
        break;
    case A_RESIZE:
        a.kind = AttrKind::Resize;
        a.axis = static_cast<int32_t>(t.u32(0));
        break;
    default:
        break;
    }
    return a;
}

// src/ir.rs:616-671
BasicBlock parse_block(const Table& b)
{
    BasicBlock blk;
    blk.name = b.str(0);
    {
        auto [s, n] = b.vec(2, 4);
        for (uint32_t i = 0; i < n; i++) {
            Table t = b.sub(s + 4 * i);
            TensorDef d;
            d.name = t.str(0);
            d.shape = t.i32vec(1);
            d.dtype = dtype_from_code(t.u32(2));
            d.has_data = t.has(3);
            if (d.has_data)
                d.data = t.bytevec(3);
            d.is_variable = t.boolean(4);
            blk.tensors.push_back(std::move(d));
        }
    }
    {
        // SHAPE values become SHAPE tensors of shape [rank] (src/ir.rs:637-652).
        auto [s, n] = b.vec(5, 4);
        for (uint32_t i = 0; i < n; i++) {
            Table t = b.sub(s + 4 * i);
            TensorDef d;
            d.name = t.str(0);
            d.shape = {static_cast<int32_t>(t.u32(1))};
            d.dtype = DT_SHAPE;
            d.has_data = t.has(2);
            if (d.has_data)
                d.data = t.bytevec(2);
            blk.tensors.push_back(std::move(d));
        }
    }
    {
        auto [s, n] = b.vec(1, 4);
        for (uint32_t i = 0; i < n; i++) {
            Table o = b.sub(s + 4 * i);
            Operator op;
            op.op = o.u32(0);
            op.inputs = o.strvec(3);
            op.outputs = o.strvec(4);
            op.attr = parse_attribute(o);
            blk.operators.push_back(std::move(op));
        }
    }
    blk.inputs = b.strvec(3);
    blk.outputs = b.strvec(4);
    return blk;
}

}  // namespace

Graph Graph::from_flatbuffer(const uint8_t* data, size_t len)
{
    if (data == nullptr || len < 8)
        throw Error(ERR_DESERIALIZE, "failed to deserialize flatbuffer: buffer too small");
    Reader r(data, len);
    Table g(r, r.deref(0));
    if (!g.has(0))
        throw Error(ERR_DESERIALIZE, "failed to deserialize flatbuffer: missing required field TosaGraph.version");
    Table version = g.sub(g.field(0));
    (void)version;
    Graph graph;
    auto [s, n] = g.vec(1, 4);
    for (uint32_t i = 0; i < n; i++) {
        Table rt = g.sub(s + 4 * i);
        Region reg;
        reg.name = rt.str(0);
        auto [bs, bn] = rt.vec(1, 4);
        for (uint32_t j = 0; j < bn; j++)
            reg.blocks.push_back(parse_block(rt.sub(bs + 4 * j)));
        graph.regions.push_back(std::move(reg));
    }
    return graph;
}

const BasicBlock* Graph::main_block() const
{
    if (regions.empty() || regions[0].blocks.empty())
        return nullptr;
    return &regions[0].blocks[0];
}

const BasicBlock* Graph::find_block(const std::string& name) const
{
    for (const auto& r : regions)
        for (const auto& b : r.blocks)
            if (b.name == name)
                return &b;
    for (const auto& r : regions)
        if (r.name == name && !r.blocks.empty())
            return &r.blocks[0];
    return nullptr;
}

}  // namespace tosa
