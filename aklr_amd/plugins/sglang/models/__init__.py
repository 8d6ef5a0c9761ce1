"""sglang model routes: the sglang functions whose work this library's ops take over."""
