"""`python -m custom_cuda_kernals_amd.cli`."""

from custom_cuda_kernals_amd.cli import main

if __name__ == "__main__":
    main()
