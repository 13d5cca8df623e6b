// Per-thread status text shared by every C ABI entry point (o2mi_last_error).
#pragma once

#include <string>

std::string& o2mi_error_slot();
