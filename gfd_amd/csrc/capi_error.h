#pragma once
// Per-thread error message behind gfd_last_error(), shared by every
// translation unit that implements a C-ABI entry point.
void gfd_internal_set_error(const char* what);
