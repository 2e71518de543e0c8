// Arrow IPC stream codec for relations of UInt32 columns (host code).
//
// The reference moves relations in and out through arrow-rs' StreamReader /
// StreamWriter (from_arrow_ipc_stream / to_arrow_ipc_stream,
// crates/xlog-cuda/src/provider/io.rs:697-773): one Schema message, exactly
// one RecordBatch, the end-of-stream marker.  This is a self-contained reader
// and writer of that format for the column type every relation on this path
// has (UInt32), with no Arrow library: the reader parses the flatbuffer
// metadata with bounds checks on every access (the input is untrusted) and
// returns pointers to the column buffers inside the stream, so the device
// upload copies each column once, straight from the caller's bytes.
//
// Format (Arrow columnar spec, "IPC streaming format"; Message.fbs and
// Schema.fbs): each message is 0xFFFFFFFF, an int32 metadata length, a
// flatbuffer Message padded to 8 bytes, then bodyLength bytes of body.  A
// flatbuffer table starts with an int32 offset back to its vtable (uint16
// vtable size, table size, then one uint16 offset per field, 0 = absent);
// references to tables, vectors and strings are uint32 offsets forward from
// the referencing field.
#include "internal.hpp"

#include <cstring>

namespace xh {

namespace {

[[noreturn]] void bad(const std::string &what) {
    throw Error{XLOG_HIP_INVALID_ARG, "arrow ipc: " + what};
}

// Message.fbs / Schema.fbs field numbers (a union field takes two slots:
// its type, then the value)
enum { MSG_VERSION = 0, MSG_HEADER_TYPE = 1, MSG_HEADER = 2, MSG_BODY_LENGTH = 3 };
enum { HDR_SCHEMA = 1, HDR_DICTIONARY_BATCH = 2, HDR_RECORD_BATCH = 3 };
enum { SCHEMA_ENDIANNESS = 0, SCHEMA_FIELDS = 1 };
enum { FIELD_NAME = 0, FIELD_NULLABLE = 1, FIELD_TYPE_TYPE = 2, FIELD_TYPE = 3, FIELD_DICTIONARY = 4, FIELD_CHILDREN = 5 };
enum { TYPE_INT = 2 };
enum { INT_BIT_WIDTH = 0, INT_IS_SIGNED = 1 };
enum { RB_LENGTH = 0, RB_NODES = 1, RB_BUFFERS = 2, RB_COMPRESSION = 3 };
constexpr int16_t METADATA_V4 = 3, METADATA_V5 = 4;
constexpr uint32_t CONTINUATION = 0xFFFFFFFFu;

// ---- reading ---------------------------------------------------------------
struct Fb {
    const uint8_t *b;
    uint64_t n;
    template <typename T>
    T get(uint64_t off) const {
        if (off > n || n - off < sizeof(T)) bad("metadata access out of bounds");
        T v;
        std::memcpy(&v, b + off, sizeof(T));
        return v;
    }
};

struct Table {
    const Fb *fb = nullptr;
    uint64_t pos = 0, vt = 0;
    uint16_t vt_size = 0;
    Table() = default;
    Table(const Fb *f, uint64_t p) : fb(f), pos(p) {
        const int64_t vt_pos = (int64_t)p - (int64_t)f->get<int32_t>(p);
        if (vt_pos < 0 || (uint64_t)vt_pos >= f->n) bad("vtable out of bounds");
        vt = (uint64_t)vt_pos;
        vt_size = f->get<uint16_t>(vt);
        if (vt_size < 4 || vt_size % 2) bad("malformed vtable");
    }
    // absolute position of field `id`, 0 when absent
    uint64_t field(int id) const {
        const uint64_t slot = 4 + 2 * (uint64_t)id;
        if (slot + 2 > vt_size) return 0;
        const uint16_t off = fb->get<uint16_t>(vt + slot);
        return off ? pos + off : 0;
    }
    template <typename T>
    T scalar(int id, T dflt) const {
        const uint64_t p = field(id);
        return p ? fb->get<T>(p) : dflt;
    }
    // target of the uoffset in field `id`, 0 when absent
    uint64_t ref(int id) const {
        const uint64_t p = field(id);
        if (!p) return 0;
        const uint64_t t = p + fb->get<uint32_t>(p);
        if (t >= fb->n) bad("reference out of bounds");
        return t;
    }
    bool has(int id) const { return field(id) != 0; }
    Table table(int id) const {
        const uint64_t t = ref(id);
        if (!t) bad("missing table");
        return Table(fb, t);
    }
};

// vector at `pos`: element count and first element position
struct Vec {
    uint64_t count = 0, first = 0;
};
Vec vec_at(const Fb &fb, uint64_t pos, uint64_t elem_size) {
    Vec v;
    if (!pos) return v;
    v.count = fb.get<uint32_t>(pos);
    v.first = pos + 4;
    if (v.count > (fb.n - v.first) / elem_size) bad("vector out of bounds");
    return v;
}

std::string string_at(const Fb &fb, uint64_t pos) {
    if (!pos) return std::string();
    const uint32_t len = fb.get<uint32_t>(pos);
    if (len > fb.n - pos - 4) bad("string out of bounds");
    return std::string(reinterpret_cast<const char *>(fb.b + pos + 4), len);
}

struct Message {
    Table msg;
    uint8_t header_type = 0;
    Table header;
    int64_t body_length = 0;
    const uint8_t *body = nullptr;
};

// Reads the message at *off; false at the end-of-stream marker.
bool next_message(const uint8_t *s, uint64_t len, uint64_t *off, Fb *fb, Message *m) {
    if (len - *off < 4) bad("truncated stream (missing end-of-stream marker)");
    uint32_t word;
    std::memcpy(&word, s + *off, 4);
    *off += 4;
    if (word == CONTINUATION) {
        if (len - *off < 4) bad("truncated stream");
        std::memcpy(&word, s + *off, 4);
        *off += 4;
    }
    const int32_t meta_len = (int32_t)word;  // pre-0.15 streams have no continuation marker
    if (meta_len == 0) return false;
    if (meta_len < 0 || (uint64_t)meta_len > len - *off) bad("metadata length out of bounds");
    fb->b = s + *off;
    fb->n = (uint64_t)meta_len;
    *off += (uint64_t)meta_len;
    const uint32_t root = fb->get<uint32_t>(0);
    m->msg = Table(fb, root);
    const int16_t version = m->msg.scalar<int16_t>(MSG_VERSION, 0);
    if (version != METADATA_V4 && version != METADATA_V5) bad("unsupported metadata version " + std::to_string(version));
    m->header_type = m->msg.scalar<uint8_t>(MSG_HEADER_TYPE, 0);
    m->header = m->msg.table(MSG_HEADER);
    m->body_length = m->msg.scalar<int64_t>(MSG_BODY_LENGTH, 0);
    if (m->body_length < 0 || (uint64_t)m->body_length > len - *off) bad("message body out of bounds");
    m->body = s + *off;
    *off += (uint64_t)m->body_length;
    return true;
}

// ---- writing ---------------------------------------------------------------
// A front-to-back flatbuffer writer: each table is written as its vtable
// followed by the table; referenced objects are appended after the
// referencing table and the uint32 offsets patched (they point forward, as
// the format requires).
class FbOut {
  public:
    std::vector<uint8_t> b;
    void align(uint64_t a) {
        while (b.size() % a) b.push_back(0);
    }
    template <typename T>
    void put_at(uint64_t pos, T v) {
        std::memcpy(b.data() + pos, &v, sizeof(T));
    }
    template <typename T>
    uint64_t put(T v) {
        align(sizeof(T));
        const uint64_t p = b.size();
        b.resize(p + sizeof(T));
        put_at(p, v);
        return p;
    }
    struct F {
        int id;
        int size;  // 1, 2, 4 or 8 bytes; 4 for an offset
        uint64_t value;
    };
    // Writes a table with the given fields (in layout order); returns the
    // positions of the fields by id (for offset patching) in `at`.
    uint64_t table(const std::vector<F> &fields, std::vector<uint64_t> &at) {
        int max_id = -1;
        for (const F &f : fields) max_id = std::max(max_id, f.id);
        const uint16_t vt_size = (uint16_t)(4 + 2 * (max_id + 1));
        align(2);
        const uint64_t vt = b.size();
        b.resize(vt + vt_size, 0);
        // the table: soffset to the vtable, then the fields, each aligned to its size
        align(8);
        if ((b.size() + 4) % 8) b.resize(b.size() + 4, 0);  // so 8-byte fields after the soffset can be aligned
        const uint64_t tab = put<int32_t>(0);
        put_at<int32_t>(tab, (int32_t)(tab - vt));
        at.assign(max_id + 1, 0);
        for (const F &f : fields) {
            uint64_t p;
            switch (f.size) {
                case 1: p = put<uint8_t>((uint8_t)f.value); break;
                case 2: p = put<uint16_t>((uint16_t)f.value); break;
                case 4: p = put<uint32_t>((uint32_t)f.value); break;
                default: p = put<uint64_t>(f.value); break;
            }
            at[f.id] = p;
            put_at<uint16_t>(vt + 4 + 2 * f.id, (uint16_t)(p - tab));
        }
        align(4);
        put_at<uint16_t>(vt, vt_size);
        put_at<uint16_t>(vt + 2, (uint16_t)(b.size() - tab));
        return tab;
    }
    void link(uint64_t field_pos, uint64_t target) { put_at<uint32_t>(field_pos, (uint32_t)(target - field_pos)); }
    // vector header (count) such that the elements after it are aligned to elem_align
    uint64_t vec(uint32_t count, uint64_t elem_align) {
        align(4);
        while ((b.size() + 4) % elem_align) b.push_back(0);
        return put<uint32_t>(count);
    }
    uint64_t str(const std::string &s) {
        const uint64_t p = put<uint32_t>((uint32_t)s.size());
        b.insert(b.end(), s.begin(), s.end());
        b.push_back(0);
        return p;
    }
};

// One encapsulated message: continuation, metadata length, the flatbuffer
// (root offset + Message table + header) padded to 8, then the body.
void emit_message(std::vector<uint8_t> &out, const FbOut &fb, const std::vector<uint8_t> &body) {
    uint64_t meta = fb.b.size();
    while ((8 + meta) % 8) ++meta;
    const uint32_t cont = CONTINUATION, ml = (uint32_t)meta;
    const uint64_t p = out.size();
    out.resize(p + 8 + meta, 0);
    std::memcpy(out.data() + p, &cont, 4);
    std::memcpy(out.data() + p + 4, &ml, 4);
    std::memcpy(out.data() + p + 8, fb.b.data(), fb.b.size());
    out.insert(out.end(), body.begin(), body.end());
}

// Message table with a header of type `htype`; returns the header field position
uint64_t message_table(FbOut &fb, uint8_t htype, int64_t body_length, uint64_t *header_field) {
    fb.put<uint32_t>(0);  // root offset, patched below
    std::vector<uint64_t> at;
    const uint64_t m = fb.table({{MSG_BODY_LENGTH, 8, (uint64_t)body_length},
                                 {MSG_HEADER, 4, 0},
                                 {MSG_VERSION, 2, (uint64_t)METADATA_V5},
                                 {MSG_HEADER_TYPE, 1, htype}},
                                at);
    fb.put_at<uint32_t>(0, (uint32_t)m);
    *header_field = at[MSG_HEADER];
    return m;
}

}  // namespace

void ipc_decode_u32(const uint8_t *s, uint64_t len, IpcColumns &out) {
    XH_REQUIRE(s || len == 0, XLOG_HIP_INVALID_ARG, "arrow ipc: stream is NULL");
    out = IpcColumns();
    uint64_t off = 0;
    Fb fb{nullptr, 0};
    Message m;
    if (!next_message(s, len, &off, &fb, &m) || m.header_type != HDR_SCHEMA) bad("stream does not start with a schema");
    // schema: every field a non-dictionary UInt32, little-endian
    const Table &schema = m.header;
    XH_REQUIRE(schema.scalar<int16_t>(SCHEMA_ENDIANNESS, 0) == 0, XLOG_HIP_UNSUPPORTED,
               "arrow ipc: big-endian streams are not supported");
    const Vec fields = vec_at(fb, schema.ref(SCHEMA_FIELDS), 4);
    XH_REQUIRE(fields.count >= 1 && fields.count <= 4, XLOG_HIP_UNSUPPORTED,
               "arrow ipc: a relation has 1..4 columns (stream has " + std::to_string(fields.count) + ")");
    out.arity = (uint32_t)fields.count;
    for (uint64_t i = 0; i < fields.count; ++i) {
        const uint64_t fp = fields.first + 4 * i;
        const Table f(&fb, fp + fb.get<uint32_t>(fp));
        const std::string name = string_at(fb, f.ref(FIELD_NAME));
        const uint8_t tt = f.scalar<uint8_t>(FIELD_TYPE_TYPE, 0);
        bool u32 = false;
        if (tt == TYPE_INT) {
            const Table it = f.table(FIELD_TYPE);
            u32 = it.scalar<int32_t>(INT_BIT_WIDTH, 0) == 32 && !it.scalar<uint8_t>(INT_IS_SIGNED, 0);
        }
        XH_REQUIRE(u32, XLOG_HIP_TYPE_MISMATCH,
                   "arrow ipc: column '" + name + "' is not UInt32 (relations on this path are u32 columns)");
        XH_REQUIRE(!f.has(FIELD_DICTIONARY), XLOG_HIP_UNSUPPORTED, "arrow ipc: dictionary-encoded columns are not supported");
        out.names.push_back(name);
    }
    // exactly one record batch (io.rs:721-737)
    bool have_batch = false;
    for (;;) {
        const uint64_t before = off;
        Fb bfb{nullptr, 0};
        Message bm;
        if (!next_message(s, len, &off, &bfb, &bm)) break;
        (void)before;
        XH_REQUIRE(bm.header_type != HDR_DICTIONARY_BATCH, XLOG_HIP_UNSUPPORTED,
                   "arrow ipc: dictionary batches are not supported");
        if (bm.header_type != HDR_RECORD_BATCH) bad("unexpected message type " + std::to_string(bm.header_type));
        XH_REQUIRE(!have_batch, XLOG_HIP_INVALID_ARG,
                   "Arrow IPC stream contains multiple record batches; this API expects exactly one");
        have_batch = true;
        const Table &rb = bm.header;
        XH_REQUIRE(!rb.has(RB_COMPRESSION), XLOG_HIP_UNSUPPORTED, "arrow ipc: compressed record batches are not supported");
        const int64_t rows = rb.scalar<int64_t>(RB_LENGTH, 0);
        if (rows < 0) bad("negative row count");
        const Vec nodes = vec_at(bfb, rb.ref(RB_NODES), 16);
        const Vec bufs = vec_at(bfb, rb.ref(RB_BUFFERS), 16);
        if (nodes.count != out.arity || bufs.count != 2ull * out.arity) bad("record batch does not match the schema");
        out.rows = (uint64_t)rows;
        out.cols.assign(out.arity, nullptr);
        for (uint32_t c = 0; c < out.arity; ++c) {
            const int64_t node_len = bfb.get<int64_t>(nodes.first + 16 * c);
            if (node_len != rows) bad("column length differs from the batch length");
            // buffer 2c is the validity bitmap; values are taken as stored, as the reference does
            // (io.rs:651-653 reads values() and ignores validity)
            const int64_t boff = bfb.get<int64_t>(bufs.first + 16 * (2 * c + 1));
            const int64_t blen = bfb.get<int64_t>(bufs.first + 16 * (2 * c + 1) + 8);
            if (boff < 0 || blen < 0 || boff > bm.body_length || blen > bm.body_length - boff) bad("column buffer out of bounds");
            if ((uint64_t)blen < 4ull * (uint64_t)rows) bad("column buffer shorter than the batch");
            out.cols[c] = bm.body + boff;
        }
    }
    XH_REQUIRE(have_batch, XLOG_HIP_INVALID_ARG, "Arrow IPC stream contained no record batches");
}

std::vector<uint8_t> ipc_encode_u32(const uint32_t *const *cols, uint32_t arity, uint64_t rows,
                                    const char *const *names) {
    XH_REQUIRE(arity >= 1 && arity <= 4, XLOG_HIP_INVALID_ARG, "arrow ipc: arity must be 1..4");
    XH_REQUIRE(rows <= (uint64_t)INT64_MAX / 4, XLOG_HIP_CAPACITY_OVERFLOW, "arrow ipc: too many rows");
    std::vector<uint8_t> out;
    // ---- schema message
    {
        FbOut fb;
        uint64_t hdr;
        message_table(fb, HDR_SCHEMA, 0, &hdr);
        std::vector<uint64_t> at;
        const uint64_t schema = fb.table({{SCHEMA_FIELDS, 4, 0}, {SCHEMA_ENDIANNESS, 2, 0}}, at);
        fb.link(hdr, schema);
        const uint64_t fv = fb.vec(arity, 4);
        fb.link(at[SCHEMA_FIELDS], fv);
        std::vector<uint64_t> slots(arity);
        for (uint32_t i = 0; i < arity; ++i) slots[i] = fb.put<uint32_t>(0);
        for (uint32_t i = 0; i < arity; ++i) {
            std::vector<uint64_t> fa;
            const uint64_t f = fb.table({{FIELD_NAME, 4, 0},
                                         {FIELD_TYPE, 4, 0},
                                         {FIELD_CHILDREN, 4, 0},
                                         {FIELD_TYPE_TYPE, 1, TYPE_INT},
                                         {FIELD_NULLABLE, 1, 0}},
                                        fa);
            fb.link(slots[i], f);
            const std::string nm = names && names[i] ? std::string(names[i]) : "c" + std::to_string(i);
            fb.link(fa[FIELD_NAME], fb.str(nm));
            std::vector<uint64_t> ia;
            const uint64_t it = fb.table({{INT_BIT_WIDTH, 4, 32}, {INT_IS_SIGNED, 1, 0}}, ia);
            fb.link(fa[FIELD_TYPE], it);
            fb.link(fa[FIELD_CHILDREN], fb.vec(0, 4));
        }
        emit_message(out, fb, {});
    }
    // ---- record batch: per column an empty validity buffer and the values, 64-byte aligned
    {
        const uint64_t col_bytes = 4 * rows, padded = (col_bytes + 63) / 64 * 64;
        FbOut fb;
        uint64_t hdr;
        message_table(fb, HDR_RECORD_BATCH, (int64_t)(padded * arity), &hdr);
        std::vector<uint64_t> at;
        const uint64_t rb = fb.table({{RB_LENGTH, 8, rows}, {RB_NODES, 4, 0}, {RB_BUFFERS, 4, 0}}, at);
        fb.link(hdr, rb);
        fb.link(at[RB_NODES], fb.vec(arity, 8));
        for (uint32_t i = 0; i < arity; ++i) {
            fb.put<uint64_t>(rows);  // FieldNode.length
            fb.put<uint64_t>(0);     // FieldNode.null_count
        }
        fb.link(at[RB_BUFFERS], fb.vec(2 * arity, 8));
        for (uint32_t i = 0; i < arity; ++i) {
            fb.put<uint64_t>(padded * i);  // validity: absent (no nulls)
            fb.put<uint64_t>(0);
            fb.put<uint64_t>(padded * i);  // values
            fb.put<uint64_t>(col_bytes);
        }
        std::vector<uint8_t> body(padded * arity, 0);
        for (uint32_t i = 0; i < arity && rows; ++i) {
            XH_REQUIRE(cols && cols[i], XLOG_HIP_INVALID_ARG, "arrow ipc: column pointer is NULL");
            std::memcpy(body.data() + padded * i, cols[i], col_bytes);
        }
        emit_message(out, fb, body);
    }
    // ---- end of stream
    const uint32_t eos[2] = {CONTINUATION, 0u};
    out.insert(out.end(), reinterpret_cast<const uint8_t *>(eos), reinterpret_cast<const uint8_t *>(eos) + 8);
    return out;
}

}  // namespace xh
