"""TEST-ONLY: vllm.envs whitelist table."""
import os

environment_variables = {"VLLM_HOST_IP": lambda: os.environ.get("VLLM_HOST_IP", "")}
