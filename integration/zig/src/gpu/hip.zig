//! src/gpu/hip.zig -- Tomoul's MI355X (gfx950) matmul backend, libtomoul_hip.so.
//!
//! The binding a Tomoul checkout adds next to src/core/blas.zig, in the same
//! pattern (src/core/blas.zig:24-54): `extern "c"` declarations of the C ABI
//! in include/tomoul_hip.h, then thin wrappers over Zig slices.  Each wrapper
//! returns true when the GPU ran the call; false means "take the CPU path"
//! (no device, or the call failed), as the HAL does for its GPU backends
//! (src/gpu/hal.zig:145-161).  Selected at build time by -Dhip=true
//! (integration/zig/build_hip.zig) and called from the comptime branches in
//! src/core/ops.zig and src/core/quantization.zig (see INTEGRATION.md).
//!
//! Every declaration below mirrors one in include/tomoul_hip.h; a CPU test
//! (tests/test_zig_shim.py) checks names, arity, integer widths and pointer
//! constness against the header.

// Status codes (TML_OK = 0, negative = error).
pub const TML_OK: c_int = 0;
pub const TML_ERR_NO_DEVICE: c_int = -6;

// Weight formats (= the .tl quant-format byte, src/core/loader.zig:23-29).
pub const FMT_F32: c_int = 0;
pub const FMT_Q8_0: c_int = 1;
pub const FMT_Q4_0: c_int = 2;
pub const FMT_Q8_K: c_int = 3;
pub const FMT_F16: c_int = 4;
pub const FMT_Q8_0_PC: c_int = 17;
pub const FMT_Q4_0_PC: c_int = 18;

// Activations fused after the bias.
pub const ACT_NONE: c_int = 0;
pub const ACT_GELU_ERF: c_int = 1; // ops.geluExact
pub const ACT_GELU_TANH: c_int = 2; // ops.gelu

/// Opaque handles of the C ABI.
pub const Prepared = ?*anyopaque; // tml_prepared_t
pub const TlFile = ?*anyopaque; // tml_tl_t

// ------------------------------------------------------------ setup
pub extern "c" fn tml_hip_init() c_int;
pub extern "c" fn tml_hip_shutdown() void;
pub extern "c" fn tml_hip_last_error() [*:0]const u8;
pub extern "c" fn tml_hip_device_name(buf: [*]u8, len: usize) c_int;

// ------------------------------------------------- host-pointer API
pub extern "c" fn tml_hip_sgemm(M: i64, N: i64, K: i64, A: [*]const f32, B: [*]const f32, C: [*]f32, alpha: f32, beta: f32) c_int;
pub extern "c" fn tml_hip_sgemm_bias(M: i64, N: i64, K: i64, A: [*]const f32, B: [*]const f32, bias: [*]const f32, C: [*]f32) c_int;
pub extern "c" fn tml_hip_sgemv(M: i64, N: i64, A: [*]const f32, x: [*]const f32, y: [*]f32, alpha: f32, beta: f32) c_int;
pub extern "c" fn tml_hip_sgemm_q8(M: i64, N: i64, K: i64, A: [*]const f32, Bq: [*]const i8, scale: f32, C: [*]f32) c_int;
pub extern "c" fn tml_hip_sgemm_q8k(M: i64, N: i64, K: i64, A: [*]const f32, Bq: [*]const i8, scales: [*]const f32, block: i64, C: [*]f32) c_int;
pub extern "c" fn tml_hip_sgemm_q4(M: i64, N: i64, K: i64, A: [*]const f32, Bp: [*]const u8, scale: f32, C: [*]f32) c_int;
pub extern "c" fn tml_hip_sgemm_f16(M: i64, N: i64, K: i64, A: [*]const f32, Bh: [*]const u16, C: [*]f32) c_int;
pub extern "c" fn tml_hip_gemm(fmt: c_int, M: i64, N: i64, K: i64, A: [*]const f32, B: *const anyopaque, scale: f32, scales: ?[*]const f32, block: i64, bias: ?[*]const f32, C: [*]f32) c_int;
pub extern "c" fn tml_hip_gemm_act(fmt: c_int, M: i64, N: i64, K: i64, A: [*]const f32, B: *const anyopaque, scale: f32, scales: ?[*]const f32, block: i64, bias: ?[*]const f32, act: c_int, C: [*]f32) c_int;
pub extern "c" fn tml_hip_gemm_residual(fmt: c_int, M: i64, N: i64, K: i64, A: [*]const f32, B: *const anyopaque, scale: f32, scales: ?[*]const f32, block: i64, bias: ?[*]const f32, residual: [*]const f32, C: [*]f32) c_int;
pub extern "c" fn tml_hip_quantize(fmt: c_int, n: i64, w: [*]const f32, q: *anyopaque, scales: ?[*]f32) c_int;
pub extern "c" fn tml_hip_weight_register(host: *const anyopaque, bytes: usize) c_int;
pub extern "c" fn tml_hip_weight_release(host: *const anyopaque) c_int;

// ----------------------------------------------- device-pointer API
pub extern "c" fn tml_hip_gemm_dev(fmt: c_int, M: i64, N: i64, K: i64, A: [*]const f32, B: *const anyopaque, scale: f32, scales: ?[*]const f32, block: i64, bias: ?[*]const f32, C: [*]f32, alpha: f32, beta: f32, stream: ?*anyopaque) c_int;
pub extern "c" fn tml_hip_gemm_ex_dev(fmt: c_int, M: i64, N: i64, K: i64, A: [*]const f32, B: *const anyopaque, scale: f32, scales: ?[*]const f32, block: i64, bias: ?[*]const f32, residual: ?[*]const f32, act: c_int, C: [*]f32, alpha: f32, beta: f32, stream: ?*anyopaque) c_int;
/// The allocation-free form of tml_hip_gemm_ex_dev (static split-K scratch of
/// TML_NOALLOC_SCRATCH_BYTES per GPU; for code under graph capture).
pub extern "c" fn tml_hip_gemm_ex_dev_noalloc(fmt: c_int, M: i64, N: i64, K: i64, A: [*]const f32, B: *const anyopaque, scale: f32, scales: ?[*]const f32, block: i64, bias: ?[*]const f32, residual: ?[*]const f32, act: c_int, C: [*]f32, alpha: f32, beta: f32, stream: ?*anyopaque) c_int;
pub extern "c" fn tml_hip_quantize_dev(fmt: c_int, n: i64, w: [*]const f32, q: *anyopaque, scales: ?[*]f32, stream: ?*anyopaque) c_int;
pub extern "c" fn tml_hip_quantize_cols_dev(fmt: c_int, K: i64, N: i64, w: [*]const f32, q: *anyopaque, scales: [*]f32, stream: ?*anyopaque) c_int;
pub extern "c" fn tml_hip_quantize_cols(fmt: c_int, K: i64, N: i64, w: [*]const f32, q: *anyopaque, scales: [*]f32) c_int;
/// Read floor of the decoder GEMVs (a measurement aid, no reference counterpart).
pub extern "c" fn tml_hip_stream_read_dev(src: *const anyopaque, bytes: i64, chunks_per_lane: c_int, out: [*]f32, stream: ?*anyopaque) c_int;

// -------------------------------------------------- prepared weights
pub extern "c" fn tml_hip_prepare_dev(fmt: c_int, K: i64, N: i64, B: *const anyopaque, scale: f32, stream: ?*anyopaque, out: *Prepared) c_int;
pub extern "c" fn tml_hip_prepare_ex_dev(fmt: c_int, K: i64, N: i64, B: *const anyopaque, scale: f32, scales: ?[*]const f32, stream: ?*anyopaque, out: *Prepared) c_int;
pub extern "c" fn tml_hip_gemm_prepared(w: Prepared, M: i64, A: [*]const f32, bias: ?[*]const f32, C: [*]f32, alpha: f32, beta: f32, stream: ?*anyopaque) c_int;
pub extern "c" fn tml_hip_prepare_rows_dev(fmt: c_int, K: i64, N: i64, W: *const anyopaque, ldw: i64, scale: f32, stream: ?*anyopaque, out: *Prepared) c_int;
pub extern "c" fn tml_hip_prepared_free(w: Prepared) c_int;
pub extern "c" fn tml_hip_gemm_prepared_ex(w: Prepared, M: i64, A: [*]const f32, bias: ?[*]const f32, residual: ?[*]const f32, act: c_int, C: [*]f32, alpha: f32, beta: f32, stream: ?*anyopaque) c_int;

// --------------------------------------------------------- .tl files
pub extern "c" fn tml_tl_open(path: [*:0]const u8, out: *TlFile) c_int;
pub extern "c" fn tml_tl_open_bytes(data: *const anyopaque, size: u64, out: *TlFile) c_int;
pub extern "c" fn tml_tl_close(f: TlFile) c_int;
pub extern "c" fn tml_tl_format(f: TlFile) c_int;
pub extern "c" fn tml_tl_count(f: TlFile) i64;
pub extern "c" fn tml_tl_name(f: TlFile, i: i64) ?[*:0]const u8;
pub extern "c" fn tml_tl_info(f: TlFile, name: [*:0]const u8, dims: ?[*]i64, cap: c_int, ndim: ?*c_int, offset: ?*u64, size: ?*u64) c_int;
pub extern "c" fn tml_tl_read(f: TlFile, name: [*:0]const u8, getter: c_int, data: ?*anyopaque, scales: ?[*]f32, scale: ?*f32) c_int;
pub extern "c" fn tml_tl_read_dev(f: TlFile, name: [*:0]const u8, getter: c_int, data: ?*anyopaque, scales: ?[*]f32, scale: ?*f32, stream: ?*anyopaque) c_int;
pub extern "c" fn tml_tl_read_dequantized_dev(f: TlFile, name: [*:0]const u8, out: [*]f32, stream: ?*anyopaque) c_int;
pub extern "c" fn tml_hip_transpose_requant_dev(fmt: c_int, rows: i64, cols: i64, q: *const anyopaque, scales: ?[*]const f32, scale: f32, q_out: *anyopaque, scales_out: [*]f32, stream: ?*anyopaque) c_int;

// ------------------------------------------------------------ wrappers
// The slices are the Tensor.data of the reference's callers
// (src/core/tensor.zig:12-18): row-major A[m,k], B[k,n] ([in, out]),
// C[m,n], preallocated by the caller and written with beta = 0.

pub fn sgemm(m: usize, n: usize, k: usize, a: []const f32, b: []const f32, c: []f32, alpha: f32, beta: f32) bool {
    return tml_hip_sgemm(@intCast(m), @intCast(n), @intCast(k), a.ptr, b.ptr, c.ptr, alpha, beta) == TML_OK;
}

pub fn sgemmBias(m: usize, n: usize, k: usize, a: []const f32, b: []const f32, bias: []const f32, c: []f32) bool {
    return tml_hip_sgemm_bias(@intCast(m), @intCast(n), @intCast(k), a.ptr, b.ptr, bias.ptr, c.ptr) == TML_OK;
}

pub fn sgemv(m: usize, n: usize, a: []const f32, x: []const f32, y: []f32, alpha: f32, beta: f32) bool {
    return tml_hip_sgemv(@intCast(m), @intCast(n), a.ptr, x.ptr, y.ptr, alpha, beta) == TML_OK;
}

pub fn sgemmQ8(m: usize, n: usize, k: usize, a: []const f32, q: []const i8, scale: f32, c: []f32) bool {
    return tml_hip_sgemm_q8(@intCast(m), @intCast(n), @intCast(k), a.ptr, q.ptr, scale, c.ptr) == TML_OK;
}

pub fn sgemmQ8K(m: usize, n: usize, k: usize, a: []const f32, q: []const i8, scales: []const f32, block: usize, c: []f32) bool {
    return tml_hip_sgemm_q8k(@intCast(m), @intCast(n), @intCast(k), a.ptr, q.ptr, scales.ptr, @intCast(block), c.ptr) == TML_OK;
}

pub fn sgemmQ4(m: usize, n: usize, k: usize, a: []const f32, packed_q: []const u8, scale: f32, c: []f32) bool {
    return tml_hip_sgemm_q4(@intCast(m), @intCast(n), @intCast(k), a.ptr, packed_q.ptr, scale, c.ptr) == TML_OK;
}

pub fn sgemmF16(m: usize, n: usize, k: usize, a: []const f32, h: []const u16, c: []f32) bool {
    return tml_hip_sgemm_f16(@intCast(m), @intCast(n), @intCast(k), a.ptr, h.ptr, c.ptr) == TML_OK;
}

/// Call once per weight at load: the weights are immutable afterwards
/// (src/core/attention.zig:54-86), so the device copy is found by pointer.
pub fn registerWeight(bytes: []const u8) bool {
    return tml_hip_weight_register(bytes.ptr, bytes.len) == TML_OK;
}

pub fn releaseWeight(bytes: []const u8) void {
    _ = tml_hip_weight_release(bytes.ptr);
}

/// fc1 + bias + GELU (erf form) in one launch (src/models/whisper/encoder.zig:244-247).
pub fn linearGeluExact(m: usize, n: usize, k: usize, a: []const f32, w: []const f32, bias: []const f32, c: []f32) bool {
    return tml_hip_gemm_act(FMT_F32, @intCast(m), @intCast(n), @intCast(k), a.ptr, w.ptr, 1.0, null, 0, bias.ptr, ACT_GELU_ERF, c.ptr) == TML_OK;
}

/// fc2 + bias + residual in one launch (src/models/whisper/encoder.zig:249-253).
pub fn linearResidual(m: usize, n: usize, k: usize, a: []const f32, w: []const f32, bias: []const f32, res: []const f32, c: []f32) bool {
    return tml_hip_gemm_residual(FMT_F32, @intCast(m), @intCast(n), @intCast(k), a.ptr, w.ptr, 1.0, null, 0, bias.ptr, res.ptr, c.ptr) == TML_OK;
}
