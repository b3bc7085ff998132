// The engine's error record: the message of the last failed call on this
// thread, which vgx_engine_last_error returns (libvgx's own when empty).
#pragma once

#include <string>

int engine_fail(int status, const std::string& msg);
void engine_clear_error();
const std::string& engine_error();
