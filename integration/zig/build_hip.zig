//! build_hip.zig -- the -Dhip build option for a Tomoul checkout.
//!
//! Import this file from build.zig and call `addHipOption` where the other
//! backend options are declared and passed to the ops and quantization
//! modules (the use_blas / use_zblas pattern).  It declares -Dhip (default
//! off) and -Dhip-lib-dir, puts `use_hip` into the given build_options, and
//! when enabled builds src/gpu/hip.zig as a module linked against
//! libtomoul_hip.so and adds it to each consumer module as "hip.zig".
//!
//!     const hip_build = @import("build_hip.zig");
//!     hip_build.addHipOption(b, target, optimize, ops_options, &.{ ops_module, quantization_module });
//!
//! The consumers then branch at comptime, before their zblas / blas
//! branches (INTEGRATION.md lists the call sites):
//!
//!     const use_hip = if (@hasDecl(build_options, "use_hip")) build_options.use_hip else false;
//!     const hip = if (use_hip) @import("hip.zig") else struct {};
const std = @import("std");

pub fn addHipOption(
    b: *std.Build,
    target: std.Build.ResolvedTarget,
    optimize: std.builtin.OptimizeMode,
    options: *std.Build.Step.Options,
    consumers: []const *std.Build.Module,
) void {
    const use_hip = b.option(bool, "hip", "Use the MI355X HIP matmul backend (libtomoul_hip.so)") orelse false;
    options.addOption(bool, "use_hip", use_hip);
    if (!use_hip) return;
    const lib_dir = b.option([]const u8, "hip-lib-dir", "Directory holding libtomoul_hip.so") orelse "tomoul_amd";
    const hip_module = b.createModule(.{
        .root_source_file = b.path("src/gpu/hip.zig"),
        .target = target,
        .optimize = optimize,
    });
    hip_module.addLibraryPath(.{ .cwd_relative = lib_dir });
    hip_module.linkSystemLibrary("tomoul_hip", .{});
    hip_module.link_libc = true;
    for (consumers) |m| m.addImport("hip.zig", hip_module);
}
