// The chat command (chat.cpp:1043-1045): hipllm_chat --gpu --model MODEL.gguf
#include "../../../include/hipllm.h"

int main(int argc, char** argv) { return hipllm_chat_main(argc, argv); }
