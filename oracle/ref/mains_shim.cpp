// Exposes the reference's two remaining CPU self-test programs
// (cpu_fufft.cpp, cpu_inplace.cpp) as callable entry points.  Each source is
// compiled where it lies in its own translation unit (see oracle/Makefile).
#if defined(FUFFT_REF_FUFFT)
#include "cpu_fufft.cpp"
extern "C" int ref_fufft_main(void) { char a0[] = "cpu_fufft"; char* argv[] = {a0, nullptr}; return fufft_ref_fufft_main(1, argv); }
#elif defined(FUFFT_REF_INPLACE)
#include "cpu_inplace.cpp"
extern "C" int ref_inplace_main(void) { return fufft_ref_inplace_main(); }
#endif
