// emulation: no half-precision intrinsics are needed
