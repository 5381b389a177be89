/* LLVM's maxnum on runtime operands: the intrinsic Rust's f32::max lowers to
 * (core::f32::max calls intrinsics::maxnumf32, emitted as llvm.maxnum.f32).
 * Built with this image's clang, where __builtin_fmaxf becomes the same
 * llvm.maxnum.f32 and is lowered by the same x86-64 backend (cmpunordss to
 * pick the non-NaN operand, maxss for the rest). glibc's fmaxf is a different
 * routine with a different signed-zero tie, so it is not used here.
 *
 * TEST INFRASTRUCTURE ONLY: it pins the oracle's max_f32 tie
 * (src/payload/elementary.rs:137-139). */
__attribute__((noinline)) float probe_maxnum(float a, float b) { return __builtin_fmaxf(a, b); }
